/**
 * @file activation.hpp
 * @brief Activation base (ref: include/CppNet/activations/activation.hpp:11-19),
 *        plus a rank-agnostic DeviceTensor overload pair.
 */
#ifndef CPPNET_ACTIVATIONS_ACTIVATION_HPP
#define CPPNET_ACTIVATIONS_ACTIVATION_HPP

#include "CppNet/core/tensor.hpp"

namespace CppNet
{
    namespace Activations
    {
        class Activation
        {
        public:
            virtual Tensor<float, 2> forward(const Tensor<float, 2>& pre_activation);
            virtual Tensor<float, 2> backward(const Tensor<float, 2>& grad_output);
            virtual Tensor<float, 4> forward(const Tensor<float, 4>& pre_activation);
            virtual Tensor<float, 4> backward(const Tensor<float, 4>& grad_output);
            virtual DeviceTensor forward(const DeviceTensor& pre_activation) = 0;
            virtual DeviceTensor backward(const DeviceTensor& grad_output) = 0;
            virtual ~Activation() = default;
        };

        /// Elementwise activation whose backward reads the cached OUTPUT.
        class OutputCachedActivation : public Activation
        {
        public:
            using Activation::forward;
            using Activation::backward;
            DeviceTensor forward(const DeviceTensor& pre_activation) override;
            DeviceTensor backward(const DeviceTensor& grad_output) override;
            const DeviceTensor& output_cache() const { return out_cache_; }
            /// The output of a forward computed elsewhere (a producing GEMM's
            /// fused epilogue), cached as forward() would cache it.
            void set_output_cache(const DeviceTensor& y) { out_cache_ = y; }

        protected:
            explicit OutputCachedActivation(const char* name) : name_(name) {}
            virtual int launch_forward(const float* x, float* y, int64_t n) = 0;
            virtual int launch_backward(const float* y, const float* dy, float* dx, int64_t n) = 0;

        private:
            const char* name_;
            DeviceTensor out_cache_;
        };
    } // namespace Activations
} // namespace CppNet
#endif
