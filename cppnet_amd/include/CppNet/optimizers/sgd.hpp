/**
 * @file sgd.hpp
 * @brief SGD on device "gpu" (ref: include/CppNet/optimizers/sgd.hpp:27, src/CppNet/optimizers/sgd.cpp:54-68).
 *
 * W -= lr g.  gpu_block_size is accepted for the reference's signature; the
 * multi-tensor kernel chooses its own launch shape.
 */
#ifndef CPPNET_OPTIMIZERS_SGD_HPP
#define CPPNET_OPTIMIZERS_SGD_HPP

#include <string>

#include "CppNet/optimizers/device_optimizer.hpp"

namespace CppNet
{
    namespace Optimizers
    {
        class SGD : public DeviceOptimizer
        {
        public:
            SGD(const std::string& device = "gpu", int gpu_block_size = 256);
            int get_gpu_block_size() const { return block_; }

        private:
            int block_;
        };
    } // namespace Optimizers
} // namespace CppNet
#endif
