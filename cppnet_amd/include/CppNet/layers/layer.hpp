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

            /// True while the gradient buffers hold no gradient of the current
            /// step: they are cleared lazily, and a backward over them writes
            /// instead of accumulating.  A captured step graph sets it after
            /// each replay to what the captured backward left, since a replay
            /// runs device work only.
            bool grads_pending_zero() const { return grads_zero_; }
            void set_grads_pending_zero(bool z) { grads_zero_ = z; }

        protected:
            bool grads_zero_ = true;
        };

        /// The backend implements device "gpu" only; any other string throws
        /// std::runtime_error("Unknown device: ...") as the reference does for
        /// unknown devices (linear.cpp:191).
        void require_gpu_device(const std::string& device, const std::string& who);
    } // namespace Layers
} // namespace CppNet
#endif
