/**
 * @file mae.hpp
 * @brief Mean absolute error, device "gpu"
 *        (ref: include/CppNet/losses/mae.hpp:27-28, src/CppNet/losses/mae.cpp:102-160).
 *
 * loss = sum |p - t| (/ element count for "mean"); grad = sign(p - t) (/ count).
 */
#ifndef CPPNET_LOSSES_MAE_HPP
#define CPPNET_LOSSES_MAE_HPP

#include "CppNet/losses/loss.hpp"

namespace CppNet
{
    namespace Losses
    {
        class MAE : public Loss
        {
        public:
            explicit MAE(const std::string& reduction = "mean", const std::string& device = "gpu");
            using Loss::forward;
            using Loss::backward;
            DeviceScalar forward(const DeviceTensor& predictions, const DeviceTensor& targets) override;
            DeviceTensor backward(const DeviceTensor& predictions, const DeviceTensor& targets) override;
            static void set_num_threads(int) {}

        private:
            std::string reduction_;
            std::string device_;
        };
    } // namespace Losses
} // namespace CppNet
#endif
