// Adam on device (ref: src/CppNet/optimizers/adam.cpp:98-133).
#include "CppNet/optimizers/adam.hpp"

#include <cmath>
#include <stdexcept>

#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Optimizers
    {
        Adam::Adam(float beta1, float beta2, float epsilon, const std::string& device)
            : beta1_(beta1), beta2_(beta2), epsilon_(epsilon), device_(device)
        {
            Layers::require_gpu_device(device_, "Adam");
        }

        void Adam::update(float* weights, const float* gradients, int size, float learning_rate)
        {
            update(weights, gradients, static_cast<int64_t>(size), learning_rate);
        }

        void Adam::update(float* weights, const float* gradients, int64_t size, float learning_rate)
        {
            if (size <= 0) return;
            if (pending_.empty()) reconcile_withheld();  // before any t of this group advances
            auto it = states_.find(weights);
            if (it == states_.end())
            {
                if (!cnhip_is_device_pointer(weights) || !cnhip_is_device_pointer(gradients))
                    throw std::invalid_argument(
                        "Adam::update: parameters and gradients must be device memory in the gpu backend");
                State s;
                s.m = DeviceTensor::zeros({size});
                s.v = DeviceTensor::zeros({size});
                it = states_.emplace(weights, std::move(s)).first;
            }
            State& s = it->second;
            if (s.m.size() != size)
                throw std::invalid_argument("Adam::update: parameter size changed for an existing key");
            ++s.t;
            // adam.cpp:121-122, evaluated identically (float pow of float t)
            const float bc1 = 1.0f - std::pow(beta1_, static_cast<float>(s.t));
            const float bc2 = 1.0f - std::pow(beta2_, static_cast<float>(s.t));
            pending_.push_back(Pending{weights, gradients, &s, size, bc1, bc2, learning_rate});
            if (group_depth_ == 0) flush();
        }

        void Adam::begin_group() { ++group_depth_; }

        void Adam::end_group()
        {
            if (group_depth_ > 0 && --group_depth_ == 0) flush();
        }

        void Adam::reconcile_withheld()
        {
            const int64_t taken = cnhip_update_faults_taken();
            if (taken == faults_seen_) return;
            faults_seen_ = taken;
            for (auto it = launched_.begin(); it != launched_.end();)
            {
                if (cnhip_update_withheld(it->seq))
                {
                    for (State* s : it->keys) --s->t;
                    it = launched_.erase(it);
                }
                else
                    ++it;
            }
        }

        void Adam::flush()
        {
            size_t i = 0;
            while (i < pending_.size())
            {
                // one fused launch per run of equal learning rates (<= 64 tensors each)
                float* W[64];
                const float* G[64];
                float* M[64];
                float* V[64];
                int64_t N[64];
                float B1[64], B2[64];
                const float lr = pending_[i].lr;
                int count = 0;
                while (i < pending_.size() && count < 64 && pending_[i].lr == lr)
                {
                    const Pending& p = pending_[i++];
                    W[count] = p.w; G[count] = p.g; M[count] = p.s->m.data(); V[count] = p.s->v.data();
                    N[count] = p.n; B1[count] = p.bc1; B2[count] = p.bc2;
                    ++count;
                }
                int st = cnhip_adam_step_multi(count, W, G, M, V, N, B1, B2, lr, beta1_, beta2_, epsilon_,
                                               Device::stream());
                if (st != CNHIP_OK)
                {
                    pending_.clear();
                    Device::check(st, "Adam::update");
                }
                Launched l{cnhip_update_seq_last(), {}};
                for (size_t k = i - count; k < i; ++k) l.keys.push_back(pending_[k].s);
                launched_.push_back(std::move(l));
                if (launched_.size() > kLaunchHistory) launched_.pop_front();
            }
            pending_.clear();
        }

        void Adam::prepare_external(const std::vector<std::pair<float*, int64_t>>& params,
                                    std::vector<float*>& m, std::vector<float*>& v, std::vector<float>& bc1,
                                    std::vector<float>& bc2)
        {
            if (!pending_.empty() || group_depth_ != 0)
                throw std::logic_error("Adam::prepare_external inside an update group");
            reconcile_withheld();  // before any t advances, as update() does
            external_.clear();
            m.clear(); v.clear(); bc1.clear(); bc2.clear();
            for (const auto& p : params)
            {
                auto it = states_.find(p.first);
                if (it == states_.end())
                {
                    State s;
                    s.m = DeviceTensor::zeros({p.second});
                    s.v = DeviceTensor::zeros({p.second});
                    it = states_.emplace(p.first, std::move(s)).first;
                }
                State& s = it->second;
                if (s.m.size() != p.second)
                    throw std::invalid_argument("Adam::prepare_external: parameter size changed for an existing key");
                external_.push_back(&s);
                m.push_back(s.m.data());
                v.push_back(s.v.data());
            }
            // t advances only once every key is known to be valid
            for (State* s : external_)
            {
                ++s->t;
                bc1.push_back(1.0f - std::pow(beta1_, static_cast<float>(s->t)));
                bc2.push_back(1.0f - std::pow(beta2_, static_cast<float>(s->t)));
            }
        }

        void Adam::commit_external()
        {
            Launched l{cnhip_update_seq_last(), external_};
            launched_.push_back(std::move(l));
            if (launched_.size() > kLaunchHistory) launched_.pop_front();
            external_.clear();
        }

        void Adam::abort_external()
        {
            for (State* s : external_) --s->t;
            external_.clear();
        }

        int Adam::step_count(const float* weights) const
        {
            auto it = states_.find(weights);
            return it == states_.end() ? 0 : it->second.t;
        }
        const DeviceTensor& Adam::first_moment(const float* weights) const
        {
            auto it = states_.find(weights);
            if (it == states_.end()) throw std::out_of_range("Adam: no state for this parameter");
            return it->second.m;
        }
        const DeviceTensor& Adam::second_moment(const float* weights) const
        {
            auto it = states_.find(weights);
            if (it == states_.end()) throw std::out_of_range("Adam: no state for this parameter");
            return it->second.v;
        }

        bool Adam::get_state(const float* weights, int64_t n, std::vector<std::vector<float>>& tensors,
                             int& t) const
        {
            auto it = states_.find(weights);
            if (it == states_.end()) return false;
            if (it->second.m.size() != n) throw std::invalid_argument("Adam::get_state: size mismatch");
            tensors.assign(2, std::vector<float>(static_cast<size_t>(n)));
            it->second.m.copy_to_host(tensors[0].data());
            it->second.v.copy_to_host(tensors[1].data());
            t = it->second.t;
            return true;
        }

        void Adam::set_state(const float* weights, int64_t n, const std::vector<std::vector<float>>& tensors,
                             int t)
        {
            if (tensors.size() != 2 || static_cast<int64_t>(tensors[0].size()) != n ||
                static_cast<int64_t>(tensors[1].size()) != n || t < 0)
                throw std::invalid_argument("Adam::set_state: expected m and v of the parameter's size");
            if (!cnhip_is_device_pointer(weights))
                throw std::invalid_argument("Adam::set_state: parameters must be device memory");
            auto it = states_.find(weights);
            if (it == states_.end())
            {
                State s;
                s.m = DeviceTensor::empty({n});
                s.v = DeviceTensor::empty({n});
                it = states_.emplace(weights, std::move(s)).first;
            }
            if (it->second.m.size() != n) throw std::invalid_argument("Adam::set_state: size mismatch");
            it->second.m.copy_from_host(tensors[0].data());
            it->second.v.copy_from_host(tensors[1].data());
            it->second.t = t;
        }
    } // namespace Optimizers
} // namespace CppNet
