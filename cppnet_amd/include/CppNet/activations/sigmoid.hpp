/**
 * @file sigmoid.hpp
 * @brief Sigmoid activation, device "gpu" (ref include/CppNet/activations/sigmoid.hpp; y = 1/(1+exp(-clamp(x,+-500))), dX = dY*(y(1-y)) (sigmoid.cpp:97-231)).
 */
#ifndef CPPNET_ACTIVATIONS_SIGMOID_HPP
#define CPPNET_ACTIVATIONS_SIGMOID_HPP

#include <string>

#include "CppNet/activations/activation.hpp"

namespace CppNet
{
    namespace Activations
    {
        class Sigmoid : public OutputCachedActivation
        {
        public:
            explicit Sigmoid(const std::string& device = "gpu");
            static void set_num_threads(int) {}

        protected:
            int launch_forward(const float* x, float* y, int64_t n) override;
            int launch_backward(const float* y, const float* dy, float* dx, int64_t n) override;
        };
    } // namespace Activations
} // namespace CppNet
#endif
