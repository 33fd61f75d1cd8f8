/**
 * @file mrs_prop.hpp
 * @brief RMSProp on device "gpu" (ref: include/CppNet/optimizers/mrs_prop.hpp:27-28, src/CppNet/optimizers/mrs_prop.cpp:83-106).
 *
 * s = rho s + (1 - rho) g g; W -= lr g / (sqrt(s) + eps).
 */
#ifndef CPPNET_OPTIMIZERS_MRS_PROP_HPP
#define CPPNET_OPTIMIZERS_MRS_PROP_HPP

#include <string>

#include "CppNet/optimizers/device_optimizer.hpp"

namespace CppNet
{
    namespace Optimizers
    {
        class RMSProp : public DeviceOptimizer
        {
        public:
            RMSProp(float rho = 0.9f, float epsilon = 1e-8f, const std::string& device = "gpu");
            float get_rho() const { return rho_; }

        private:
            float rho_;
        };
    } // namespace Optimizers
} // namespace CppNet
#endif
