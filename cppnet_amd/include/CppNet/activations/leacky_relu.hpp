/**
 * @file leacky_relu.hpp
 * @brief LeakyReLU, device "gpu" (ref: include/CppNet/activations/leacky_relu.hpp:34,
 *        src/CppNet/activations/leacky_relu.cpp:93-229).
 *
 * y = x > 0 ? x : alpha x; the backward reads the cached INPUT:
 * dx = x > 0 ? dy : alpha dy.  Any rank (the reference has 2-D and 4-D).
 */
#ifndef CPPNET_ACTIVATIONS_LEACKY_RELU_HPP
#define CPPNET_ACTIVATIONS_LEACKY_RELU_HPP

#include <string>

#include "CppNet/activations/activation.hpp"

namespace CppNet
{
    namespace Activations
    {
        class LeakyReLU : public Activation
        {
        public:
            explicit LeakyReLU(float alpha = 0.01f, const std::string& device = "gpu");
            using Activation::forward;
            using Activation::backward;
            DeviceTensor forward(const DeviceTensor& pre_activation) override;
            DeviceTensor backward(const DeviceTensor& grad_output) override;
            float get_alpha() const { return alpha_; }
            static void set_num_threads(int) {}

        private:
            float alpha_;
            DeviceTensor in_cache_;
        };
    } // namespace Activations
} // namespace CppNet
#endif
