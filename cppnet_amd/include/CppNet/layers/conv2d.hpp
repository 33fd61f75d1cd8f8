/**
 * @file conv2d.hpp
 * @brief Conv2D, device "gpu" (ref: include/CppNet/layers/conv2d.hpp:41-43,
 *        src/CppNet/layers/conv2d.cpp:29-213).
 *
 * Input [N, C, H, W] ColMajor, weights [OC, C, KS, KS], output
 * [N, OC, HO, WO] with HO = (H + 2*padding - KS)/stride + 1.  Weights start
 * xavier-uniform with fans C*KS^2 and OC*KS^2 (conv2d.cpp:42-50), biases 0.
 * backward() OVERWRITES the gradients (conv2d.cpp:149-152) and always
 * returns dX; step() updates W then b and then clears the gradients
 * (conv2d.cpp:200-213).  Runs as implicit-GEMM MFMA kernels.
 */
#ifndef CPPNET_LAYERS_CONV2D_HPP
#define CPPNET_LAYERS_CONV2D_HPP

#include <string>

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"
#include "CppNet/layers/max_pool2d.hpp"

namespace CppNet
{
    namespace Layers
    {
        class Conv2D : public Layer
        {
        public:
            Conv2D(int in_channels, int out_channels, int kernel_size, int stride = 1,
                   int padding = 0, bool bias = true, const std::string& device = "gpu");

            Tensor<float, 4> forward(const Tensor<float, 4>& input);
            Tensor<float, 4> backward(const Tensor<float, 4>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            /// forward() followed by ReLU, in the GEMM epilogue; returns the
            /// ReLU output (what the ReLU's backward reads).
            DeviceTensor forward_relu(const DeviceTensor& input);
            /// forward_relu() followed by `pool`'s forward, in one call where
            /// the shape allows: returns the pooled output and records the
            /// forward in `pool` (MaxPool2D::set_fused_forward).
            DeviceTensor forward_relu_maxpool(const DeviceTensor& input, MaxPool2D& pool);
            DeviceTensor backward(const DeviceTensor& grad_output);
            /// backward() with the input gradient optional: input_grad = false
            /// computes the parameter gradients only and returns an undefined
            /// tensor (a model's first layer, whose input is data).
            DeviceTensor backward(const DeviceTensor& grad_output, bool input_grad);
            /// Whether backward_params_maxpool_relu serves `pool` (a forward
            /// fused by forward_relu_maxpool into it, with a shape that fits).
            bool fuses_pool_backward(const DeviceTensor& grad_pooled, const MaxPool2D& pool) const;
            /// The parameter gradients of this layer, its ReLU and `pool`
            /// from the pooled gradient in one pass (no input gradient, no
            /// gradient of the conv output stored): equal to pool's
            /// backward_relu_pooled() then backward(g, false).
            void backward_params_maxpool_relu(const DeviceTensor& grad_pooled, const MaxPool2D& pool);

            bool is_trainable() const override { return trainable_; }
            void step(Optimizers::Optimizer& optimizer, float learning_rate) override;
            void reset_grads() override { grads_zero_ = true; }
            void freeze() { trainable_ = false; }
            void unfreeze() { trainable_ = true; }

            const Tensor<float, 4> get_weights() const;
            const Tensor<float, 1> get_biases() const;
            const Tensor<float, 4> get_grad_weights() const;
            const Tensor<float, 1> get_grad_biases() const;
            void set_weights(const Tensor<float, 4>& weights);
            void set_biases(const Tensor<float, 1>& biases);
            DeviceTensor& weights() { return W_; }
            DeviceTensor& biases() { return b_; }
            DeviceTensor& grad_weights() { materialize_grads(); return gW_; }
            DeviceTensor& grad_biases() { materialize_grads(); return gb_; }

            int get_in_channels() const { return in_channels_; }
            int get_out_channels() const { return out_channels_; }
            int get_kernel_size() const { return kernel_size_; }
            int get_stride() const { return stride_; }
            int get_padding() const { return padding_; }
            bool has_bias() const { return bias_flag_; }
            void set_max_batch_size(int) {}

        private:
            void materialize_grads() const;
            DeviceTensor forward_impl(const DeviceTensor& input, bool relu);
            int in_channels_, out_channels_, kernel_size_, stride_, padding_;
            bool bias_flag_;
            bool trainable_ = true;
            std::string device_;
            DeviceTensor W_, b_, gW_, gb_, in_cache_;
        };
    } // namespace Layers
} // namespace CppNet
#endif
