/**
 * @file rnn.hpp
 * @brief Elman RNN, device "gpu" (ref: include/CppNet/layers/rnn.hpp:40-41,
 *        src/CppNet/layers/rnn.cpp:27-191).
 *
 * X [B, S, I] -> Y [B, S, H] (the full sequence), h_0 = 0,
 * h_t = tanh(x_t W_ih + h_{t-1} W_hh + b).  W_ih [I, H], W_hh [H, H] xavier
 * uniform, b = 0 (rnn.cpp:27-46).  backward() overwrites the grads; step()
 * updates W_ih, W_hh, b and clears them (rnn.cpp:173-184).
 */
#ifndef CPPNET_LAYERS_RNN_HPP
#define CPPNET_LAYERS_RNN_HPP

#include "CppNet/layers/lstm.hpp"

namespace CppNet
{
    namespace Layers
    {
        class RNN : public RecurrentBase
        {
        public:
            RNN(int input_size, int hidden_size, bool return_sequences = true,
                const std::string& device = "gpu");
            Tensor<float, 3> forward(const Tensor<float, 3>& input);
            Tensor<float, 3> backward(const Tensor<float, 3>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);
            DeviceTensor backward(const DeviceTensor& grad_output, bool input_grad);
        };
    } // namespace Layers
} // namespace CppNet
#endif
