/**
 * @file relu.hpp
 * @brief ReLU activation, device "gpu" (ref include/CppNet/activations/relu.hpp; y = max(x,0), dX = dY*(y>0) (relu.cpp:97-225)).
 */
#ifndef CPPNET_ACTIVATIONS_RELU_HPP
#define CPPNET_ACTIVATIONS_RELU_HPP

#include <string>

#include "CppNet/activations/activation.hpp"

namespace CppNet
{
    namespace Activations
    {
        class ReLU : public OutputCachedActivation
        {
        public:
            explicit ReLU(const std::string& device = "gpu");
            static void set_num_threads(int) {}

        protected:
            int launch_forward(const float* x, float* y, int64_t n) override;
            int launch_backward(const float* y, const float* dy, float* dx, int64_t n) override;
        };
    } // namespace Activations
} // namespace CppNet
#endif
