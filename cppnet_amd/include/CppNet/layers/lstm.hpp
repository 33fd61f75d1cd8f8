/**
 * @file lstm.hpp
 * @brief LSTM, device "gpu" (ref: include/CppNet/layers/lstm.hpp:53-54,
 *        src/CppNet/layers/lstm.cpp:34-266).
 *
 * Input [B, S, I], output [B, S, H] ColMajor (the full sequence: the
 * reference ignores return_sequences).  Gate column blocks i, f, g, o; W_ih,
 * W_hh xavier-uniform with limits sqrt(6/(I+H)) and sqrt(6/2H); bias 0 except
 * the forget block = 1 (lstm.cpp:42-51); h0 = c0 = 0.  backward() overwrites
 * the grads; step() updates W_ih, W_hh, b then clears them (lstm.cpp:255-266).
 * The forward caches (gate activations, c, tanh c) stay in HBM.
 */
#ifndef CPPNET_LAYERS_LSTM_HPP
#define CPPNET_LAYERS_LSTM_HPP

#include <string>

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Layers
    {
        /// Shared state of the recurrent layers (gates = 4 for LSTM, 3 for GRU).
        class RecurrentBase : public Layer
        {
        public:
            bool is_trainable() const override { return trainable_; }
            void step(Optimizers::Optimizer& optimizer, float learning_rate) override;
            void reset_grads() override { grads_zero_ = true; }
            void freeze() { trainable_ = false; }
            void unfreeze() { trainable_ = true; }
            int get_input_size() const { return input_size_; }
            int get_hidden_size() const { return hidden_size_; }
            bool get_return_sequences() const { return return_sequences_; }

            /// Host copies (the reference returns references to host tensors).
            const Tensor<float, 2> get_W_ih() const { return W_ih_.to_host<float, 2>(); }
            const Tensor<float, 2> get_W_hh() const { return W_hh_.to_host<float, 2>(); }
            const Tensor<float, 1> get_bias() const { return b_.to_host<float, 1>(); }
            void set_W_ih(const Tensor<float, 2>& w);
            void set_W_hh(const Tensor<float, 2>& w);
            void set_bias(const Tensor<float, 1>& b);

            DeviceTensor& weights() { return W_ih_; }  ///< W_ih (first parameter)
            DeviceTensor& W_ih() { return W_ih_; }
            DeviceTensor& W_hh() { return W_hh_; }
            DeviceTensor& bias() { return b_; }
            DeviceTensor& grad_W_ih() { materialize_grads(); return gW_ih_; }
            DeviceTensor& grad_W_hh() { materialize_grads(); return gW_hh_; }
            DeviceTensor& grad_bias() { materialize_grads(); return gb_; }

        protected:
            RecurrentBase(int input_size, int hidden_size, bool return_sequences, int gates,
                          const std::string& device, const char* name);
            void check_input(const DeviceTensor& x) const;
            void materialize_grads() const;
            int input_size_, hidden_size_, gates_;
            bool return_sequences_;
            bool trainable_ = true;
            std::string device_;
            const char* name_;
            DeviceTensor W_ih_, W_hh_, b_, gW_ih_, gW_hh_, gb_;
            DeviceTensor in_cache_, out_cache_, gates_cache_;
        };

        class LSTM : public RecurrentBase
        {
        public:
            LSTM(int input_size, int hidden_size, bool return_sequences = true,
                 const std::string& device = "gpu");
            Tensor<float, 3> forward(const Tensor<float, 3>& input);
            Tensor<float, 3> backward(const Tensor<float, 3>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);
            /// backward() with the input gradient optional: input_grad = false
            /// computes the parameter gradients only and returns an undefined
            /// tensor (a model's first layer, whose input is data).
            DeviceTensor backward(const DeviceTensor& grad_output, bool input_grad);
            /// backward() for a gradient [B, H] of the last step's output only
            /// (an LSTM -> SequenceLast stack): equal to SequenceLast's backward
            /// followed by backward(), without materialising the zeros.
            DeviceTensor backward_last(const DeviceTensor& grad_last, bool input_grad);

        private:
            DeviceTensor c_cache_, tanh_c_cache_;
        };

        /**
         * GRU, device "gpu" (ref: include/CppNet/layers/gru.hpp:44-63,
         * src/CppNet/layers/gru.cpp:30-322): gate blocks z, r, n,
         * n = tanh(x W_in + (r*h) W_hn + b_n), h = (1-z) n + z h_prev; bias 0.
         */
        class GRU : public RecurrentBase
        {
        public:
            GRU(int input_size, int hidden_size, bool return_sequences = true,
                const std::string& device = "gpu");
            Tensor<float, 3> forward(const Tensor<float, 3>& input);
            Tensor<float, 3> backward(const Tensor<float, 3>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);
            /// backward() with the input gradient optional: input_grad = false
            /// computes the parameter gradients only and returns an undefined
            /// tensor (a model's first layer, whose input is data).
            DeviceTensor backward(const DeviceTensor& grad_output, bool input_grad);

        private:
            DeviceTensor rh_cache_;
        };
    } // namespace Layers
} // namespace CppNet
#endif
