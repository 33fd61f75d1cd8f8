/**
 * @file momentum.hpp
 * @brief Momentum on device "gpu" (ref: include/CppNet/optimizers/momentum.hpp:27, src/CppNet/optimizers/momentum.cpp:81-104).
 *
 * v = mu v - lr g; W += v (v per key, zero at the first update).
 */
#ifndef CPPNET_OPTIMIZERS_MOMENTUM_HPP
#define CPPNET_OPTIMIZERS_MOMENTUM_HPP

#include <string>

#include "CppNet/optimizers/device_optimizer.hpp"

namespace CppNet
{
    namespace Optimizers
    {
        class Momentum : public DeviceOptimizer
        {
        public:
            explicit Momentum(float mu = 0.9f, const std::string& device = "gpu");
            float get_mu() const { return mu_; }

        private:
            float mu_;
        };
    } // namespace Optimizers
} // namespace CppNet
#endif
