/**
 * @file global_pool.hpp
 * @brief GlobalAvgPool2D / GlobalMaxPool2D, device "gpu"
 *        (ref: include/CppNet/layers/global_pool.hpp:36, 81;
 *        src/CppNet/layers/global_pool.cpp:111-395).
 *
 * [N, C, H, W] -> [N, C].  Average: sum over h then w, times 1/(H W);
 * backward spreads dY/(H W).  Max: first maximum of a strict > scan (h outer,
 * w inner) from -inf, argmax kept as (h, w); backward routes dY there.
 */
#ifndef CPPNET_LAYERS_GLOBAL_POOL_HPP
#define CPPNET_LAYERS_GLOBAL_POOL_HPP

#include <string>
#include <vector>

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Layers
    {
        class GlobalAvgPool2D : public Layer
        {
        public:
            explicit GlobalAvgPool2D(const std::string& device = "gpu");
            Tensor<float, 2> forward(const Tensor<float, 4>& input);
            Tensor<float, 4> backward(const Tensor<float, 2>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);
            bool is_trainable() const override { return false; }
            void step(Optimizers::Optimizer&, float) override {}

        private:
            std::string device_;
            std::vector<int64_t> in_dims_;
        };

        class GlobalMaxPool2D : public Layer
        {
        public:
            explicit GlobalMaxPool2D(const std::string& device = "gpu");
            Tensor<float, 2> forward(const Tensor<float, 4>& input);
            Tensor<float, 4> backward(const Tensor<float, 2>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);
            bool is_trainable() const override { return false; }
            void step(Optimizers::Optimizer&, float) override {}
            /// argmax positions of the last forward, [N, C] ColMajor (host copies)
            std::vector<int32_t> get_argmax_h() const;
            std::vector<int32_t> get_argmax_w() const;

        private:
            std::string device_;
            std::vector<int64_t> in_dims_;
            DeviceTensor ah_, aw_;
        };
    } // namespace Layers
} // namespace CppNet
#endif
