/**
 * @file flatten.hpp
 * @brief Flatten [N, C, H, W] -> [N, C*H*W] (ref: include/CppNet/layers/flatten.hpp:25-37,
 *        src/CppNet/layers/flatten.cpp:15-39).  In ColMajor this is a
 *        reshape of the same buffer (feature = c + C*(h + H*w)); on device it
 *        is a view, no copy and no kernel.
 */
#ifndef CPPNET_LAYERS_FLATTEN_HPP
#define CPPNET_LAYERS_FLATTEN_HPP

#include <array>

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Layers
    {
        class Flatten : public Layer
        {
        public:
            Flatten() = default;
            Tensor<float, 2> forward(const Tensor<float, 4>& input);
            Tensor<float, 4> backward(const Tensor<float, 2>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);
            bool is_trainable() const override { return false; }
            void step(Optimizers::Optimizer&, float) override {}

        private:
            std::array<int64_t, 4> input_shape_{{0, 0, 0, 0}};
        };
    } // namespace Layers
} // namespace CppNet
#endif
