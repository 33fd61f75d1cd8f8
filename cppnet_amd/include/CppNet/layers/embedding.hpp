/**
 * @file embedding.hpp
 * @brief Embedding, device "gpu" (ref: include/CppNet/layers/embedding.hpp,
 *        src/CppNet/layers/embedding.cpp:33-185).
 *
 * ids [B, S] int32 -> [B, S, D] ColMajor.  Weights start U(-1/sqrt(D),
 * 1/sqrt(D)) (embedding.cpp:38-39).  An id outside [0, V) throws
 * std::out_of_range, as the cpu-eigen branch does (embedding.cpp:87-90).
 * backward() OVERWRITES grad_weight (zero, then the deterministic per-token
 * sum of the gradient rows in the reference's (n, s) order) and returns a
 * zero [B, S, D] tensor, as the reference does; step() updates the weights
 * and clears the gradient (embedding.cpp:177-185).
 *
 * In HBM the table is kept token-major (element (v, d) at d + D*v, the
 * transpose of the reference's ColMajor [V, D]) so a lookup reads one
 * contiguous row; get_weight()/set_weight() convert.
 */
#ifndef CPPNET_LAYERS_EMBEDDING_HPP
#define CPPNET_LAYERS_EMBEDDING_HPP

#include <string>

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Layers
    {
        class Embedding : public Layer
        {
        public:
            Embedding(int vocab_size, int embed_dim, const std::string& device = "gpu");

            Tensor<float, 3> forward(const Tensor<int, 2>& input);
            Tensor<float, 3> backward(const Tensor<float, 3>& grad_output);
            /// ids: int32 device tensor [B, S]; an id outside [0, V) throws
            /// (one 4-byte read-back per call).
            DeviceTensor forward(const DeviceTensor& ids);
            /// Same, for ids the caller has already checked to lie in [0, V)
            /// (e.g. when the batch was uploaded): no read-back, so the step
            /// stays asynchronous.  Out-of-range ids still produce zero rows.
            DeviceTensor forward(const DeviceTensor& ids, bool ids_checked);
            DeviceTensor backward(const DeviceTensor& grad_output);
            /// backward() with the input gradient optional: the ids are not
            /// differentiable, so the reference returns zeros
            /// (embedding.cpp:171-174); input_grad = false (a model's first
            /// layer in a training step) skips allocating and clearing them
            /// and returns an undefined tensor.
            DeviceTensor backward(const DeviceTensor& grad_output, bool input_grad);

            bool is_trainable() const override { return trainable_; }
            void step(Optimizers::Optimizer& optimizer, float learning_rate) override;
            void reset_grads() override { grads_zero_ = true; }
            void freeze() { trainable_ = false; }
            void unfreeze() { trainable_ = true; }
            int get_vocab_size() const { return vocab_size_; }
            int get_embed_dim() const { return embed_dim_; }

            /// Host copies in the reference's layout, ColMajor [V, D].
            const Tensor<float, 2> get_weight() const;
            const Tensor<float, 2> get_grad_weight() const;
            void set_weight(const Tensor<float, 2>& w);

            /// Row order of the [B, S, D] device tensors the DeviceTensor
            /// overloads take and return: 0 = the reference's (row b + B*s
            /// of [B*S, D]), 1 = by sample (row s + S*b).  For a model that
            /// owns the whole Embedding -> MeanPool1D chain (no reference
            /// counterpart); the host-Tensor overloads need order 0.
            void set_row_order(int rows);
            int get_row_order() const { return rows_; }
            /// Device tables, token-major (see above).
            DeviceTensor& weights() { return Wt_; }
            DeviceTensor& grad_weights() { materialize_grads(); return gWt_; }

        private:
            void materialize_grads() const;
            int vocab_size_, embed_dim_;
            bool trainable_ = true;
            std::string device_;
            DeviceTensor Wt_, gWt_, ids_cache_, oob_;
            int rows_ = 0;
        };
    } // namespace Layers
} // namespace CppNet
#endif
