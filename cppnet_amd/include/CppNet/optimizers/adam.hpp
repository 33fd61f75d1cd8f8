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
#include <utility>
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

            /// An update of these tensors that a fused train-step launch
            /// performs itself (cnhip_mlp2_bce_adam_step): the same
            /// bookkeeping as update() for each key (state created on first
            /// use, t advanced, bias corrections as adam.cpp:121-122),
            /// returning each key's moments and bias corrections.  Call
            /// commit_external() right after that launch, which records it
            /// for the withheld-update reconciliation as flush() does, or
            /// abort_external() when the launch was refused, which takes the
            /// step counts back.
            void prepare_external(const std::vector<std::pair<float*, int64_t>>& params,
                                  std::vector<float*>& m, std::vector<float*>& v, std::vector<float>& bc1,
                                  std::vector<float>& bc2);
            void commit_external();
            void abort_external();
            float beta1() const { return beta1_; }
            float beta2() const { return beta2_; }
            float epsilon() const { return epsilon_; }

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
            std::vector<State*> external_;    // keys of the prepared external update
            int64_t faults_seen_ = 0;
            static constexpr std::size_t kLaunchHistory = 4096;
        };
    } // namespace Optimizers
} // namespace CppNet
#endif
