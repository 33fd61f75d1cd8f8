/**
 * @file binary_cross_entropy.hpp
 * @brief BinaryCrossEntropy, device "gpu"
 *        (ref: include/CppNet/losses/binary_cross_entropy.hpp:24-25,
 *        src/CppNet/losses/binary_cross_entropy.cpp:143-225).
 *
 * p is clipped to [1e-7, 1-1e-7]; loss = mean (or sum) of
 * -[t log p + (1-t) log(1-p)]; grad = (p-t)/(p(1-p)), divided by the element
 * count for "mean".  "none" returns the mean loss and the undivided gradient,
 * as the reference does.  from_logits and pos_weight are stored and unused,
 * as in the reference.  The host overloads validate targets to {0,1} like
 * validate_inputs (101-131); the device overloads skip that check (it would
 * need a host synchronisation every step).
 */
#ifndef CPPNET_LOSSES_BCE_HPP
#define CPPNET_LOSSES_BCE_HPP

#include "CppNet/losses/loss.hpp"

namespace CppNet
{
    namespace Losses
    {
        class BinaryCrossEntropy : public Loss
        {
        public:
            BinaryCrossEntropy(const std::string& reduction = "mean", bool from_logits = false,
                               float pos_weight = 1.0f, const std::string& device = "gpu");
            using Loss::forward;
            using Loss::backward;
            float forward(const Tensor<float, 2>& predictions, const Tensor<float, 2>& targets) override;
            Tensor<float, 2> backward(const Tensor<float, 2>& predictions,
                                      const Tensor<float, 2>& targets) override;
            DeviceScalar forward(const DeviceTensor& predictions, const DeviceTensor& targets) override;
            DeviceTensor backward(const DeviceTensor& predictions, const DeviceTensor& targets) override;
            static void set_num_threads(int) {}
            /// reduction codes of the device forward ("none" returns the mean)
            /// and backward (only "mean" divides the gradient)
            int forward_reduction() const { return reduction_ == "sum" ? CNHIP_REDUCE_SUM : CNHIP_REDUCE_MEAN; }
            int backward_reduction() const { return reduction_ == "mean" ? CNHIP_REDUCE_MEAN : CNHIP_REDUCE_SUM; }

        private:
            std::string reduction_;
            bool from_logits_;
            float pos_weight_;
            std::string device_;
        };
    } // namespace Losses
} // namespace CppNet
#endif
