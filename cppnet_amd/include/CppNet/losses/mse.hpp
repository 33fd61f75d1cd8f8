/**
 * @file mse.hpp
 * @brief Mean squared error, device "gpu"
 *        (ref: include/CppNet/losses/mse.hpp:27-28, src/CppNet/losses/mse.cpp:102-161).
 *
 * loss = sum (p-t)^2, divided by the element count for "mean";
 * grad = 2(p-t), divided by the element count for "mean".
 */
#ifndef CPPNET_LOSSES_MSE_HPP
#define CPPNET_LOSSES_MSE_HPP

#include "CppNet/losses/loss.hpp"

namespace CppNet
{
    namespace Losses
    {
        class MSE : public Loss
        {
        public:
            explicit MSE(const std::string& reduction = "mean", const std::string& device = "gpu");
            using Loss::forward;
            using Loss::backward;
            DeviceScalar forward(const DeviceTensor& predictions, const DeviceTensor& targets) override;
            DeviceTensor backward(const DeviceTensor& predictions, const DeviceTensor& targets) override;
            /// forward() then backward() in one call: one launch for outputs of
            /// up to 64 Ki elements, with the same loss and gradient bits as
            /// the two calls.
            DeviceScalar forward_backward(const DeviceTensor& predictions, const DeviceTensor& targets,
                                          DeviceTensor& grad);
            static void set_num_threads(int) {}

        private:
            std::string reduction_;
            std::string device_;
        };
    } // namespace Losses
} // namespace CppNet
#endif
