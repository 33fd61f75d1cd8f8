/**
 * @file adagrad.hpp
 * @brief Adagrad on device "gpu" (ref: include/CppNet/optimizers/adagrad.hpp:27, src/CppNet/optimizers/adagrad.cpp:83-106).
 *
 * a += g g; W -= lr g / (sqrt(a) + eps).
 */
#ifndef CPPNET_OPTIMIZERS_ADAGRAD_HPP
#define CPPNET_OPTIMIZERS_ADAGRAD_HPP

#include <string>

#include "CppNet/optimizers/device_optimizer.hpp"

namespace CppNet
{
    namespace Optimizers
    {
        class Adagrad : public DeviceOptimizer
        {
        public:
            explicit Adagrad(float epsilon = 1e-8f, const std::string& device = "gpu");
            float get_epsilon() const { return eps_; }

        private:
            float eps_;
        };
    } // namespace Optimizers
} // namespace CppNet
#endif
