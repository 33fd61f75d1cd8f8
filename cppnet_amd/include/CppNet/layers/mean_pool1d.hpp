/**
 * @file mean_pool1d.hpp
 * @brief MeanPool1D, device "gpu" (ref: include/CppNet/layers/mean_pool1d.hpp,
 *        src/CppNet/layers/mean_pool1d.cpp:24-150).
 *
 * [B, S, D] -> [B, D], the mean over the sequence; backward broadcasts
 * grad / S.  No parameters.
 */
#ifndef CPPNET_LAYERS_MEAN_POOL1D_HPP
#define CPPNET_LAYERS_MEAN_POOL1D_HPP

#include <string>

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Layers
    {
        class MeanPool1D : public Layer
        {
        public:
            explicit MeanPool1D(const std::string& device = "gpu");
            Tensor<float, 2> forward(const Tensor<float, 3>& input);
            Tensor<float, 3> backward(const Tensor<float, 2>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);
            bool is_trainable() const override { return false; }
            void step(Optimizers::Optimizer&, float) override {}
            void reset_grads() override {}
            /// Row order of the [B, S, D] device tensors the DeviceTensor
            /// overloads take and return: 0 = the reference's (row b + B*s
            /// of [B*S, D]), 1 = by sample (row s + S*b).  For a model that
            /// owns the whole Embedding -> MeanPool1D chain (no reference
            /// counterpart); the host-Tensor overloads need order 0.
            void set_row_order(int rows);
            int get_row_order() const { return rows_; }

        private:
            std::string device_;
            int64_t B_ = 0, S_ = 0, D_ = 0;
            int rows_ = 0;
        };
    } // namespace Layers
} // namespace CppNet
#endif
