/**
 * @file init.hpp
 * @brief Weight initialisation (ref: include/CppNet/utils/init.hpp,
 *        src/CppNet/utils/init.cpp:15-130).
 *
 * Same methods, limits and defaults as the reference.  The reference seeds
 * its generator from std::random_device only; set_seed() makes runs
 * reproducible here (it has no reference counterpart).
 */
#ifndef CPPNET_UTILS_INIT_HPP
#define CPPNET_UTILS_INIT_HPP

#include <cstdint>
#include <string>

#include "CppNet/core/tensor.hpp"

namespace CppNet
{
    namespace Utils
    {
        void set_seed(uint64_t seed);
        /// A 64-bit value from the same generator (seeds the device-side
        /// dropout masks, so set_seed() fixes them too).
        uint64_t next_seed();
        Tensor<float, 2> xavier_uniform(int rows, int cols);
        Tensor<float, 2> xavier_normal(int rows, int cols);
        Tensor<float, 2> he_uniform(int rows, int cols);
        Tensor<float, 2> he_normal(int rows, int cols);
        Tensor<float, 2> uniform_init(int rows, int cols, float low = -1.0f, float high = 1.0f);
        Tensor<float, 2> normal_init(int rows, int cols, float mean = 0.0f, float stddev = 0.01f);
        Tensor<float, 2> constant_init(int rows, int cols, float value);
        Tensor<float, 2> init_weights(int rows, int cols, const std::string& method = "xavier");
    } // namespace Utils
} // namespace CppNet
#endif
