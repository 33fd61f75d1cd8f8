/**
 * @file gelu.hpp
 * @brief GELU, device "gpu".  The reference has no GELU; this is the exact
 *        form y = x Phi(x) = 0.5 x (1 + erf(x / sqrt 2)), with
 *        dx = dy (Phi(x) + x phi(x)).  Caches its INPUT for backward.
 */
#ifndef CPPNET_ACTIVATIONS_GELU_HPP
#define CPPNET_ACTIVATIONS_GELU_HPP

#include <string>

#include "CppNet/activations/activation.hpp"

namespace CppNet
{
    namespace Activations
    {
        class GELU : public Activation
        {
        public:
            explicit GELU(const std::string& device = "gpu");
            using Activation::forward;
            using Activation::backward;
            DeviceTensor forward(const DeviceTensor& pre_activation) override;
            DeviceTensor backward(const DeviceTensor& grad_output) override;
            const DeviceTensor& input_cache() const { return in_cache_; }
            /// The input of a forward computed elsewhere (a producing GEMM's
            /// fused epilogue), cached as forward() would cache it.
            void set_input_cache(const DeviceTensor& x) { in_cache_ = x; }

        private:
            DeviceTensor in_cache_;
        };
    } // namespace Activations
} // namespace CppNet
#endif
