/**
 * @file categorical_cross_entropy.hpp
 * @brief Categorical cross-entropy, device "gpu"
 *        (ref: include/CppNet/losses/categorical_cross_entropy.hpp:25-26,
 *        src/CppNet/losses/categorical_cross_entropy.cpp:141-424).
 *
 * Predictions [B, C] are logits (from_logits, softmax applied here) or
 * probabilities; targets one-hot / soft [B, C] or int class labels [B].
 * label_smoothing > 0 replaces t by t (1 - ls) + ls / C.  loss = sum
 * -t log(clip(p, 1e-15, 1 - 1e-15)), divided by B for "mean" ("none"
 * returns the sum, as the reference does); gradient p - t (logits) or
 * -t / clip(p), divided by B for "mean".
 */
#ifndef CPPNET_LOSSES_CATEGORICAL_CROSS_ENTROPY_HPP
#define CPPNET_LOSSES_CATEGORICAL_CROSS_ENTROPY_HPP

#include <vector>

#include "CppNet/losses/loss.hpp"

namespace CppNet
{
    namespace Losses
    {
        class CategoricalCrossEntropy : public Loss
        {
        public:
            CategoricalCrossEntropy(const std::string& reduction = "mean", bool from_logits = true,
                                    float label_smoothing = 0.0f, const std::string& device = "gpu");
            using Loss::forward;
            using Loss::backward;
            DeviceScalar forward(const DeviceTensor& predictions, const DeviceTensor& targets) override;
            DeviceTensor backward(const DeviceTensor& predictions, const DeviceTensor& targets) override;
            /// Integer class labels (one-hot built on the host, as the reference
            /// does); throws std::runtime_error for a label outside [0, C).
            float forward(const Tensor<float, 2>& predictions, const std::vector<int>& labels);
            Tensor<float, 2> backward(const Tensor<float, 2>& predictions, const std::vector<int>& labels);
            bool get_from_logits() const { return from_logits_; }
            float get_label_smoothing() const { return label_smoothing_; }
            static void set_num_threads(int) {}

        private:
            Tensor<float, 2> one_hot(const std::vector<int>& labels, int64_t B, int64_t C) const;
            std::string reduction_;
            bool from_logits_;
            float label_smoothing_;
            std::string device_;
            DeviceTensor probs_cache_, targets_cache_;
        };
    } // namespace Losses
} // namespace CppNet
#endif
