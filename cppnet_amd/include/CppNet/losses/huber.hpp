/**
 * @file huber.hpp
 * @brief Huber loss, device "gpu"
 *        (ref: include/CppNet/losses/huber.hpp:28-29, src/CppNet/losses/huber.cpp:104-178).
 *
 * Per element, d = p - t: 0.5 d^2 where |d| <= delta, else delta (|d| - delta/2);
 * grad d or delta sign(d); both / element count for "mean".
 */
#ifndef CPPNET_LOSSES_HUBER_HPP
#define CPPNET_LOSSES_HUBER_HPP

#include "CppNet/losses/loss.hpp"

namespace CppNet
{
    namespace Losses
    {
        class Huber : public Loss
        {
        public:
            explicit Huber(float delta = 1.0f, const std::string& reduction = "mean",
                           const std::string& device = "gpu");
            using Loss::forward;
            using Loss::backward;
            DeviceScalar forward(const DeviceTensor& predictions, const DeviceTensor& targets) override;
            DeviceTensor backward(const DeviceTensor& predictions, const DeviceTensor& targets) override;
            float get_delta() const { return delta_; }
            static void set_num_threads(int) {}

        private:
            float delta_;
            std::string reduction_;
            std::string device_;
        };
    } // namespace Losses
} // namespace CppNet
#endif
