/**
 * @file device_optimizer.hpp
 * @brief Shared machinery of the device SGD / Momentum / Adagrad / RMSProp
 *        (ref: src/CppNet/optimizers/{sgd,momentum,adagrad,mrs_prop}.cpp).
 *
 * State (velocity, accumulator, mean square) is kept per parameter pointer,
 * in HBM next to the parameter, zero-initialised on the key's first update,
 * as the reference keys its host vectors by the weight pointer.  Between
 * begin_group() and end_group() the updates of many tensors are queued and
 * issued as ONE multi-tensor kernel (cnhip_optimizer_step_multi).
 */
#ifndef CPPNET_OPTIMIZERS_DEVICE_OPTIMIZER_HPP
#define CPPNET_OPTIMIZERS_DEVICE_OPTIMIZER_HPP

#include <string>
#include <unordered_map>
#include <vector>

#include "CppNet/core/tensor.hpp"
#include "CppNet/optimizers/optimizer.hpp"

namespace CppNet
{
    namespace Optimizers
    {
        class DeviceOptimizer : public Optimizer
        {
        public:
            using Optimizer::update;
            void update(float* weights, const float* gradients, int size, float learning_rate) override;
            void update(float* weights, const float* gradients, int64_t size, float learning_rate) override;
            void begin_group() override;
            void end_group() override;
            /// The per-key state tensor (velocity / accumulator / mean square).
            const DeviceTensor& state(const float* weights) const;

            int kind_code() const override { return 1 + kind_; }  // 1 SGD, 2 Momentum, 3 Adagrad, 4 RMSProp
            int state_tensors() const override;
            bool get_state(const float* weights, int64_t n, std::vector<std::vector<float>>& tensors,
                           int& t) const override;
            void set_state(const float* weights, int64_t n, const std::vector<std::vector<float>>& tensors,
                           int t) override;

        protected:
            DeviceOptimizer(int kind, float hyper, float epsilon, const std::string& device, const char* name);

        private:
            struct Pending
            {
                float* w;
                const float* g;
                float* s;
                int64_t n;
                float lr;
            };
            void flush();
            int kind_;
            float hyper_, epsilon_;
            std::string device_;
            const char* name_;
            std::unordered_map<const void*, DeviceTensor> states_;
            std::vector<Pending> pending_;
            int group_depth_ = 0;
        };
    } // namespace Optimizers
} // namespace CppNet
#endif
