/**
 * @file optimizer.hpp
 * @brief Optimizer base (ref: include/CppNet/optimizers/optimizer.hpp:20-21).
 *
 * update() keeps the reference signature.  In this backend the parameter and
 * gradient pointers are DEVICE pointers (the layers' HBM-resident state);
 * passing host memory is rejected with std::invalid_argument.
 * begin_group()/end_group() let a caller (SequentialModel::update) gather the
 * updates of many tensors into one fused launch.
 */
#ifndef CPPNET_OPTIMIZERS_OPTIMIZER_HPP
#define CPPNET_OPTIMIZERS_OPTIMIZER_HPP

#include <cstdint>

namespace CppNet
{
    namespace Optimizers
    {
        class Optimizer
        {
        public:
            virtual void update(float* weights, const float* gradients, int size,
                                float learning_rate) = 0;
            virtual void update(float* weights, const float* gradients, int64_t size,
                                float learning_rate)
            {
                update(weights, gradients, static_cast<int>(size), learning_rate);
            }
            virtual void begin_group() {}
            virtual void end_group() {}
            virtual ~Optimizer() = default;
        };
    } // namespace Optimizers
} // namespace CppNet
#endif
