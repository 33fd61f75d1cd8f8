/**
 * @file softmax.hpp
 * @brief Softmax over the last dimension, device "gpu"
 *        (ref: include/CppNet/activations/softmax.hpp:35,
 *        src/CppNet/activations/softmax.cpp:105-323).
 *
 * For a 2-D [B, F] input over F, for a 4-D input over its last dimension;
 * caches the output; backward dx = y (dy - sum_j dy y).
 */
#ifndef CPPNET_ACTIVATIONS_SOFTMAX_HPP
#define CPPNET_ACTIVATIONS_SOFTMAX_HPP

#include <string>

#include "CppNet/activations/activation.hpp"

namespace CppNet
{
    namespace Activations
    {
        class Softmax : public Activation
        {
        public:
            explicit Softmax(const std::string& device = "gpu");
            using Activation::forward;
            using Activation::backward;
            DeviceTensor forward(const DeviceTensor& pre_activation) override;
            DeviceTensor backward(const DeviceTensor& grad_output) override;
            const DeviceTensor& output_cache() const { return out_cache_; }

        private:
            DeviceTensor out_cache_;
        };
    } // namespace Activations
} // namespace CppNet
#endif
