/**
 * @file dropout.hpp
 * @brief Dropout, device "gpu" (ref: include/CppNet/layers/dropout.hpp:34-76,
 *        src/CppNet/layers/dropout.cpp:15-270).
 *
 * Training: y = x * mask * 1/(1 - p), mask ~ Bernoulli(1 - p) per element;
 * backward dx = dy * mask * 1/(1 - p) with the forward's mask.  Eval mode or
 * p == 0: identity both ways.  The reference draws the mask from a
 * time-seeded host mt19937; here it is generated on the device from a
 * counter-based hash of (seed, offset), the seed taken from
 * Utils::set_seed's generator at construction and the offset advanced by the
 * element count of every forward, so runs are reproducible.
 */
#ifndef CPPNET_LAYERS_DROPOUT_HPP
#define CPPNET_LAYERS_DROPOUT_HPP

#include <cstdint>
#include <string>

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Layers
    {
        class Dropout : public Layer
        {
        public:
            explicit Dropout(float p = 0.5f, const std::string& device = "gpu");
            Tensor<float, 2> forward(const Tensor<float, 2>& input);
            Tensor<float, 4> forward(const Tensor<float, 4>& input);
            Tensor<float, 2> backward(const Tensor<float, 2>& grad_output);
            Tensor<float, 4> backward(const Tensor<float, 4>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);

            bool is_trainable() const override { return false; }
            void step(Optimizers::Optimizer&, float) override {}
            void train() { training_ = true; }
            void eval() { training_ = false; }
            bool is_training() const { return training_; }
            float get_p() const { return p_; }
            /// The last training forward's mask as 0/1 floats (host copy).
            std::vector<float> get_mask() const;
            /// The mask generator's seed and position (the element count of
            /// all training forwards so far); checkpoints save and restore them.
            uint64_t rng_seed() const { return seed_; }
            uint64_t rng_offset() const { return offset_; }
            void set_rng_state(uint64_t seed, uint64_t offset)
            {
                seed_ = seed;
                offset_ = offset;
            }

        private:
            float p_;
            bool training_ = true;
            std::string device_;
            uint64_t seed_, offset_ = 0;
            DeviceTensor mask_;   // one byte per element, packed four to a word
            int64_t mask_n_ = 0;  // element count of the last applied mask
            bool applied_ = false;  // whether the last forward applied a mask
        };
    } // namespace Layers
} // namespace CppNet
#endif
