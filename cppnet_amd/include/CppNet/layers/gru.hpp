/**
 * @file gru.hpp
 * @brief GRU, device "gpu" (ref: include/CppNet/layers/gru.hpp); declared with
 *        LSTM in lstm.hpp, which shares their recurrent base.
 */
#ifndef CPPNET_LAYERS_GRU_HPP
#define CPPNET_LAYERS_GRU_HPP
#include "CppNet/layers/lstm.hpp"
#endif
