/**
 * @file tanh.hpp
 * @brief Tanh activation, device "gpu" (ref include/CppNet/activations/tanh.hpp; y = tanh x, dX = dY*(1-y^2) (tanh.cpp:136-219)).
 */
#ifndef CPPNET_ACTIVATIONS_TANH_HPP
#define CPPNET_ACTIVATIONS_TANH_HPP

#include <string>

#include "CppNet/activations/activation.hpp"

namespace CppNet
{
    namespace Activations
    {
        class Tanh : public OutputCachedActivation
        {
        public:
            explicit Tanh(const std::string& device = "gpu");
            static void set_num_threads(int) {}

        protected:
            int launch_forward(const float* x, float* y, int64_t n) override;
            int launch_backward(const float* y, const float* dy, float* dx, int64_t n) override;
        };
    } // namespace Activations
} // namespace CppNet
#endif
