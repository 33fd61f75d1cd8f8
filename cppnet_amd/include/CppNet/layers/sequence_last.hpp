/**
 * @file sequence_last.hpp
 * @brief [B, S, D] -> [B, D]: the last time step of a sequence, and the
 *        gradient scattered back into zeros.  The reference harness writes
 *        this slice by hand after the recurrent layer
 *        (benchmarks/sequence_benckmark.cpp:152-155, 166-170); here it is a
 *        parameter-free step so a SequentialModel can chain
 *        LSTM/GRU -> SequenceLast -> Linear.  No reference class.
 */
#ifndef CPPNET_LAYERS_SEQUENCE_LAST_HPP
#define CPPNET_LAYERS_SEQUENCE_LAST_HPP

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Layers
    {
        class SequenceLast : public Layer
        {
        public:
            DeviceTensor forward(const DeviceTensor& x);
            DeviceTensor backward(const DeviceTensor& g);
            bool is_trainable() const override { return false; }
            void step(Optimizers::Optimizer&, float) override {}

        private:
            std::vector<int64_t> in_dims_;
        };
    } // namespace Layers
} // namespace CppNet
#endif
