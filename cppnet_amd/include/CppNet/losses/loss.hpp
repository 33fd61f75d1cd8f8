/**
 * @file loss.hpp
 * @brief Loss base (ref: include/CppNet/losses/loss.hpp:22-32) and the
 *        device-resident loss value.
 */
#ifndef CPPNET_LOSSES_LOSS_HPP
#define CPPNET_LOSSES_LOSS_HPP

#include <string>

#include "CppNet/core/tensor.hpp"

namespace CppNet
{
    namespace Losses
    {
        /// A loss value still in HBM.  get() (or conversion to float)
        /// synchronises the stream and reads it; holding it costs nothing.
        class DeviceScalar
        {
        public:
            DeviceScalar() = default;
            explicit DeviceScalar(DeviceTensor t) : t_(std::move(t)) {}
            float get() const;
            operator float() const { return get(); }
            const DeviceTensor& tensor() const { return t_; }

        private:
            DeviceTensor t_;
        };

        class Loss
        {
        public:
            virtual ~Loss() = default;
            /// Host overloads: one H2D of each input, then the device path.
            virtual float forward(const Tensor<float, 2>& predictions, const Tensor<float, 2>& targets);
            virtual Tensor<float, 2> backward(const Tensor<float, 2>& predictions,
                                              const Tensor<float, 2>& targets);
            virtual DeviceScalar forward(const DeviceTensor& predictions, const DeviceTensor& targets) = 0;
            virtual DeviceTensor backward(const DeviceTensor& predictions, const DeviceTensor& targets) = 0;
        };

        /// "mean" -> 0, "sum" -> 1 (the cnhip reduction codes); "none" is
        /// accepted where the reference accepts it and maps per loss.
        int reduction_code(const std::string& reduction, const char* who, bool allow_none);
    } // namespace Losses
} // namespace CppNet
#endif
