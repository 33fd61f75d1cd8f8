/**
 * @file attention.hpp
 * @brief MultiHeadAttention, device "gpu" (ref: include/CppNet/layers/
 *        attention.hpp, src/CppNet/layers/attention.cpp:35-587).
 *
 * query/key/value [B, S, D] ColMajor -> [B, S, D].  Like the reference's
 * cpu-eigen path, attention runs as ONE full-width head scaled by
 * 1/sqrt(D/num_heads) (attention.cpp:83, 187-189); there are no biases.
 * W_q, W_k, W_v, W_o [D, D] start xavier-uniform (attention.cpp:47-50).
 * backward() OVERWRITES the four gradients and returns dQ + dK + dV
 * (attention.cpp:565-567); step() updates W_q, W_k, W_v, W_o and clears the
 * gradients (attention.cpp:574-587).
 *
 * The four weights (and gradients) are views of one [D, 4D] buffer, so for
 * self-attention (query == key == value) the three projections, their weight
 * gradients and the input gradient each run as one GEMM.
 */
#ifndef CPPNET_LAYERS_ATTENTION_HPP
#define CPPNET_LAYERS_ATTENTION_HPP

#include <string>

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Layers
    {
        class MultiHeadAttention : public Layer
        {
        public:
            MultiHeadAttention(int embed_dim, int num_heads, const std::string& device = "gpu");

            Tensor<float, 3> forward(const Tensor<float, 3>& query, const Tensor<float, 3>& key,
                                     const Tensor<float, 3>& value);
            Tensor<float, 3> backward(const Tensor<float, 3>& grad_output);
            DeviceTensor forward(const DeviceTensor& query, const DeviceTensor& key,
                                 const DeviceTensor& value);
            DeviceTensor backward(const DeviceTensor& grad_output);
            /// forward(x, x, x) + residual and its backward with the skip
            /// branch's gradient added into dX, each fused into the last GEMM
            /// (equal to the separate call and add).
            DeviceTensor forward_residual(const DeviceTensor& query, const DeviceTensor& key,
                                          const DeviceTensor& value, const DeviceTensor& residual);
            DeviceTensor backward_residual(const DeviceTensor& grad_output, const DeviceTensor& skip_grad);

            bool is_trainable() const override { return trainable_; }
            void step(Optimizers::Optimizer& optimizer, float learning_rate) override;
            void reset_grads() override { grads_zero_ = true; }
            void freeze() { trainable_ = false; }
            void unfreeze() { trainable_ = true; }
            int get_embed_dim() const { return embed_dim_; }
            int get_num_heads() const { return num_heads_; }

            /// Host copies, ColMajor [D, D]; which: 0 q, 1 k, 2 v, 3 o.
            const Tensor<float, 2> get_weight(int which) const;
            const Tensor<float, 2> get_grad_weight(int which) const;
            void set_weight(int which, const Tensor<float, 2>& w);
            /// Attention weights of the last forward, [B, S, S] ColMajor (n, i, j).
            const Tensor<float, 3> get_attention_weights() const;

            /// Row order of the [B, S, D] device tensors the DeviceTensor
            /// overloads take and return: 0 = the reference's (row b + B*s
            /// of [B*S, D]), 1 = by sample (row s + S*b).  For a model that
            /// owns the whole Embedding -> MeanPool1D chain (no reference
            /// counterpart); the host-Tensor overloads need order 0.
            void set_row_order(int rows);
            int get_row_order() const { return rows_; }
            DeviceTensor& weight(int which);
            DeviceTensor& grad_weight(int which);

        private:
            void materialize_grads() const;
            int embed_dim_, num_heads_;
            bool trainable_ = true;
            std::string device_;
            DeviceTensor Wall_, gWall_;  // [D, 4D]: W_q | W_k | W_v | W_o
            DeviceTensor W_[4], gW_[4];
            DeviceTensor q_cache_, k_cache_, v_cache_, cache_;
            int rows_ = 0;
        };
    } // namespace Layers
} // namespace CppNet
#endif
