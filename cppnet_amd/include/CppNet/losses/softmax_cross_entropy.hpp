/**
 * @file softmax_cross_entropy.hpp
 * @brief Fused softmax + cross-entropy, device "gpu"
 *        (ref: include/CppNet/losses/softmax_cross_entropy.hpp:42-43,
 *        src/CppNet/losses/softmax_cross_entropy.cpp:118-195).
 *
 * Logits and targets are ColMajor [batch, classes].  forward() caches the row
 * softmax; backward() returns (softmax - targets) [/ batch for "mean"], and
 * recomputes the forward first when the cache does not match the shape, as
 * the reference does (165-170).
 */
#ifndef CPPNET_LOSSES_SOFTMAX_CE_HPP
#define CPPNET_LOSSES_SOFTMAX_CE_HPP

#include "CppNet/losses/loss.hpp"

namespace CppNet
{
    namespace Losses
    {
        class SoftmaxCrossEntropy : public Loss
        {
        public:
            explicit SoftmaxCrossEntropy(const std::string& reduction = "mean",
                                         const std::string& device = "gpu");
            using Loss::forward;
            using Loss::backward;
            DeviceScalar forward(const DeviceTensor& logits, const DeviceTensor& targets) override;
            DeviceTensor backward(const DeviceTensor& logits, const DeviceTensor& targets) override;
            const DeviceTensor& softmax_cache() const { return softmax_cache_; }
            /// forward() then backward() in one call (one launch for batches
            /// of at most 256 rows), the same values bit for bit; the
            /// gradient is written to `grad` (allocated when its shape differs)
            DeviceScalar forward_backward(const DeviceTensor& logits, const DeviceTensor& targets,
                                          DeviceTensor& grad);

        private:
            std::string reduction_;
            std::string device_;
            DeviceTensor softmax_cache_;
        };
    } // namespace Losses
} // namespace CppNet
#endif
