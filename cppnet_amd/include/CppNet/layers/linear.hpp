/**
 * @file linear.hpp
 * @brief Linear (fully connected) layer, device "gpu"
 *        (ref: include/CppNet/layers/linear.hpp, src/CppNet/layers/linear.cpp).
 *
 *   output = input * W + b       W: [in_size, out_size], b: [out_size]
 *
 * Parameters, gradients and the cached input live in HBM.  backward()
 * ADDS into grad_W / grad_b (the cpu-eigen semantics, linear.cpp:346-352);
 * reset_grads() clears them; step() never does (linear.cpp:126-146).  dX is
 * computed even for a frozen layer (linear.cpp:357).
 *
 * Host-tensor overloads copy in and out (one H2D and one D2H each); the
 * DeviceTensor overloads never touch host memory.
 */
#ifndef CPPNET_LAYERS_LINEAR_HPP
#define CPPNET_LAYERS_LINEAR_HPP

#include <string>

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Layers
    {
        class MaxPool2D;
    }
}

namespace CppNet
{
    namespace Layers
    {
        class Linear : public Layer
        {
        public:
            Linear(int in_size, int out_size, std::string layer_name = "Linear",
                   bool trainable = true, bool bias = true, std::string device = "gpu",
                   std::string weight_init = "xavier");

            Tensor<float, 2> forward(const Tensor<float, 2>& input);
            Tensor<float, 2> backward(const Tensor<float, 2>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);
            /// backward() with the input gradient optional: input_grad = false
            /// computes the parameter gradients only and returns an undefined
            /// tensor (a model's first layer, whose input is data).
            DeviceTensor backward(const DeviceTensor& grad_output, bool input_grad);
            /// forward() followed by activation act (CNHIP_ACT_RELU / _GELU) in
            /// one GEMM epilogue; returns the activation's output.  For GELU,
            /// *pre_act receives X W + b (what the GELU's backward reads).
            DeviceTensor forward_act(const DeviceTensor& input, int act,
                                     DeviceTensor* pre_act = nullptr);
            /// backward() whose input gradient also carries the derivative of
            /// activation act of the layer below: act_aux is that ReLU's output
            /// or that GELU's input.  Equals backward() then the activation's
            /// backward().
            DeviceTensor backward_act(const DeviceTensor& grad_output, int act,
                                      const DeviceTensor& act_aux);
            /// Whether backward_maxpool_relu() serves this layer: its input is
            /// the (flattened) pooled output of pool's last fused Conv2D ->
            /// ReLU -> MaxPool2D forward, and the shapes fit the one-pass kernel.
            bool fuses_maxpool_backward(const DeviceTensor& grad_output, const MaxPool2D& pool) const;
            /// backward() followed by the Flatten's, pool's and ReLU's backward
            /// of a Conv2D -> ReLU -> MaxPool2D -> Flatten -> this stack, in one
            /// pass (cnhip_linear_backward_maxpool_relu): accumulates the
            /// parameter gradients as backward() does and returns the gradient
            /// at the ReLU's input, [N, C, H, W].
            DeviceTensor backward_maxpool_relu(const DeviceTensor& grad_output, const MaxPool2D& pool);
            /// forward(input) + residual (a skip connection, [B, out]) in the
            /// GEMM epilogue; equals forward() followed by the add.  The
            /// matching backward is backward_act(g, CNHIP_ACT_RESIDUAL,
            /// skip_grad): dX = dY W^T + skip_grad.
            DeviceTensor forward_residual(const DeviceTensor& input, const DeviceTensor& residual);

            bool is_trainable() const override { return trainable_; }
            void step(Optimizers::Optimizer& optimizer, float learning_rate) override;
            void reset_grads() override;
            void freeze() { trainable_ = false; }
            void unfreeze() { trainable_ = true; }

            int get_input_size() const { return in_size_; }
            int get_output_size() const { return out_size_; }
            std::string get_layer_name() const { return layer_name_; }
            std::string get_device() const { return device_; }
            bool has_bias() const { return bias_flag_; }

            /// Host copies of the device state (synchronise the stream).
            const Tensor<float, 2> get_weights() const;
            const Tensor<float, 1> get_biases() const;
            const Tensor<float, 2> get_grad_weights() const;
            const Tensor<float, 1> get_grad_biases() const;
            void set_weights(const Tensor<float, 2>& weights);
            void set_biases(const Tensor<float, 1>& biases);

            /// Device-resident state.
            DeviceTensor& weights() { return W_; }
            DeviceTensor& biases() { return b_; }
            DeviceTensor& grad_weights() { materialize_grads(); return gW_; }
            DeviceTensor& grad_biases() { materialize_grads(); return gb_; }

            void reinitialize_weights(const std::string& method);
            /// Capacity hint of the reference gpu path (linear.cpp:460-468);
            /// buffers here are sized per call, so it only validates.
            void set_max_batch_size(int max_batch_size);
            static void set_num_threads(int) {}
            void print_layer_info() const;

        private:
            int in_size_, out_size_;
            std::string layer_name_;
            bool trainable_;
            bool bias_flag_;
            std::string device_;
            std::string weight_init_;
            DeviceTensor W_, b_, gW_, gb_;
            DeviceTensor in_cache_;
            // reset_grads() only marks the gradients as zero; the next
            // backward then writes instead of adding (0 + x == x), and any
            // reader before that gets them cleared first.
            void materialize_grads() const;
        };
    } // namespace Layers
} // namespace CppNet
#endif
