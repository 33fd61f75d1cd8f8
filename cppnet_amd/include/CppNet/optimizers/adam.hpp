/**
 * @file adam.hpp
 * @brief Adam on device (ref: include/CppNet/optimizers/adam.hpp:27-28,
 *        src/CppNet/optimizers/adam.cpp:98-133).
 *
 * State (m, v, step t) is kept per parameter pointer, as in the reference:
 * each key has its own t, and the bias corrections 1 - beta^t are computed
 * in float on the host exactly as adam.cpp:121-122 does.  m and v live in
 * HBM next to the parameters.  Between begin_group() and end_group() the
 * updates are queued and issued as ONE fused multi-tensor kernel.
 */
#ifndef CPPNET_OPTIMIZERS_ADAM_HPP
#define CPPNET_OPTIMIZERS_ADAM_HPP

#include <deque>
#include <string>
#include <unordered_map>
#include <vector>

#include "CppNet/core/tensor.hpp"
#include "CppNet/optimizers/optimizer.hpp"

namespace CppNet
{
    namespace Optimizers
    {
        class Adam : public Optimizer
        {
        public:
            Adam(float beta1 = 0.9f, float beta2 = 0.999f, float epsilon = 1e-8f,
                 const std::string& device = "gpu");
            using Optimizer::update;
            void update(float* weights, const float* gradients, int size,
                        float learning_rate) override;
            void update(float* weights, const float* gradients, int64_t size,
                        float learning_rate) override;
            void begin_group() override;
            void end_group() override;

            int step_count(const float* weights) const;
            const DeviceTensor& first_moment(const float* weights) const;
            const DeviceTensor& second_moment(const float* weights) const;

            int kind_code() const override { return 0; }
            int state_tensors() const override { return 2; }  // m, v
            bool get_state(const float* weights, int64_t n, std::vector<std::vector<float>>& tensors,
                           int& t) const override;
            void set_state(const float* weights, int64_t n, const std::vector<std::vector<float>>& tensors,
                           int t) override;
            void reconcile_withheld() override;

        private:
            struct State
            {
                DeviceTensor m, v;
                int t = 0;
            };
            struct Pending
            {
                float* w;
                const float* g;
                State* s;
                int64_t n;
                float bc1, bc2, lr;
            };
            // one fused launch: its sequence number and the keys whose t it advanced
            struct Launched
            {
                int64_t seq;
                std::vector<State*> keys;
            };
            void flush();

            float beta1_, beta2_, epsilon_;
            std::string device_;
            std::unordered_map<const void*, State> states_;
            std::vector<Pending> pending_;
            int group_depth_ = 0;
            std::deque<Launched> launched_;  // the last kLaunchHistory launches
            int64_t faults_seen_ = 0;
            static constexpr std::size_t kLaunchHistory = 4096;
        };
    } // namespace Optimizers
} // namespace CppNet
#endif
