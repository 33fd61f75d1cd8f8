/**
 * @file layer.hpp
 * @brief Layer base (ref: include/CppNet/layers/layer.hpp:15-24).
 */
#ifndef CPPNET_LAYERS_LAYER_HPP
#define CPPNET_LAYERS_LAYER_HPP

#include <string>

namespace CppNet
{
    namespace Optimizers
    {
        class Optimizer;
    }
    namespace Layers
    {
        class Layer
        {
        public:
            virtual bool is_trainable() const = 0;
            virtual void step(Optimizers::Optimizer& optimizer, float learning_rate) = 0;
            virtual void reset_grads() {}
            virtual ~Layer() = default;
        };

        /// The backend implements device "gpu" only; any other string throws
        /// std::runtime_error("Unknown device: ...") as the reference does for
        /// unknown devices (linear.cpp:191).
        void require_gpu_device(const std::string& device, const std::string& who);
    } // namespace Layers
} // namespace CppNet
#endif
