// The reference's classes off the BASELINE configs on device "gpu":
// LeakyReLU, Softmax, CategoricalCrossEntropy, MAE, Huber, SGD, Momentum,
// Adagrad, RMSProp, Dropout, GlobalAvgPool2D, GlobalMaxPool2D and the Elman
// RNN (ref: src/CppNet/activations/{leacky_relu,softmax}.cpp,
// losses/{categorical_cross_entropy,mae,huber}.cpp,
// optimizers/{sgd,momentum,adagrad,mrs_prop}.cpp,
// layers/{dropout,global_pool,rnn}.cpp).
#include <stdexcept>
#include <string>
#include <vector>

#include "CppNet/activations/leacky_relu.hpp"
#include "CppNet/activations/softmax.hpp"
#include "CppNet/layers/dropout.hpp"
#include "CppNet/layers/global_pool.hpp"
#include "CppNet/layers/rnn.hpp"
#include "CppNet/losses/categorical_cross_entropy.hpp"
#include "CppNet/losses/huber.hpp"
#include "CppNet/losses/mae.hpp"
#include "CppNet/optimizers/adagrad.hpp"
#include "CppNet/optimizers/momentum.hpp"
#include "CppNet/optimizers/mrs_prop.hpp"
#include "CppNet/optimizers/sgd.hpp"
#include "CppNet/utils/init.hpp"

namespace CppNet
{
    namespace Activations
    {
        // ---------------------------------------------------------------- LeakyReLU
        LeakyReLU::LeakyReLU(float alpha, const std::string& device) : alpha_(alpha)
        {
            Layers::require_gpu_device(device, "LeakyReLU");
        }

        DeviceTensor LeakyReLU::forward(const DeviceTensor& x)
        {
            if (!x.defined() || x.size() == 0)
                throw std::runtime_error("LeakyReLU: empty " + std::to_string(x.rank()) + "D input");
            DeviceTensor y = DeviceTensor::empty(x.dims());
            Device::check(cnhip_leaky_relu_forward(x.data(), y.data(), x.size(), alpha_, Device::stream()),
                          "LeakyReLU::forward");
            in_cache_ = x;
            return y;
        }

        DeviceTensor LeakyReLU::backward(const DeviceTensor& g)
        {
            if (!g.defined() || g.size() == 0)
                throw std::runtime_error("LeakyReLU: empty " + std::to_string(g.rank()) + "D grad");
            if (!in_cache_.defined() || in_cache_.size() != g.size())
                throw std::runtime_error("LeakyReLU: backward before forward or shape mismatch");
            DeviceTensor dx = DeviceTensor::empty(g.dims());
            Device::check(cnhip_leaky_relu_backward(in_cache_.data(), g.data(), dx.data(), g.size(), alpha_,
                                                    Device::stream()),
                          "LeakyReLU::backward");
            return dx;
        }

        // ---------------------------------------------------------------- Softmax
        Softmax::Softmax(const std::string& device) { Layers::require_gpu_device(device, "Softmax"); }

        DeviceTensor Softmax::forward(const DeviceTensor& x)
        {
            if (!x.defined() || x.size() == 0)
                throw std::runtime_error("Softmax: empty " + std::to_string(x.rank()) + "D input");
            const int64_t L = x.dimension(x.rank() - 1), R = x.size() / L;
            DeviceTensor y = DeviceTensor::empty(x.dims());
            Device::check(cnhip_softmax_forward(x.data(), y.data(), R, L, Device::stream()), "Softmax::forward");
            out_cache_ = y;
            return y;
        }

        DeviceTensor Softmax::backward(const DeviceTensor& g)
        {
            if (!g.defined() || g.size() == 0)
                throw std::runtime_error("Softmax: empty " + std::to_string(g.rank()) + "D grad");
            if (!out_cache_.defined() || out_cache_.dims() != g.dims())
                throw std::runtime_error("Softmax: backward before forward or shape mismatch");
            const int64_t L = g.dimension(g.rank() - 1), R = g.size() / L;
            DeviceTensor dx = DeviceTensor::empty(g.dims());
            Device::check(cnhip_softmax_backward(out_cache_.data(), g.data(), dx.data(), R, L, Device::stream()),
                          "Softmax::backward");
            return dx;
        }
    } // namespace Activations

    namespace Losses
    {
        // MAE and Huber divide for "mean" and sum for any other string
        // (mae.cpp:122-127, huber.cpp:134-139)
        static int mean_or_sum(const std::string& r) { return r == "mean" ? CNHIP_REDUCE_MEAN : CNHIP_REDUCE_SUM; }

        // CategoricalCrossEntropy's forward takes "mean", "sum" or "none" (the
        // sum) and throws for anything else (categorical_cross_entropy.cpp:243-257)
        static int cce_reduction(const std::string& r)
        {
            if (r == "mean") return CNHIP_REDUCE_MEAN;
            if (r == "sum" || r == "none") return CNHIP_REDUCE_SUM;
            throw std::runtime_error("CategoricalCrossEntropy: Invalid reduction type. Use 'mean', 'sum', or 'none'");
        }

        static void same_shape(const DeviceTensor& p, const DeviceTensor& t, const char* who)
        {
            if (!p.defined() || !t.defined() || p.size() == 0)
                throw std::runtime_error(std::string(who) + ": empty input tensors");
            if (p.dims() != t.dims())
                throw std::runtime_error(std::string(who) + ": predictions " + shape_str(p.dims()) +
                                         " and targets " + shape_str(t.dims()) + " shape mismatch");
        }

        // ---------------------------------------------------------------- CCE
        CategoricalCrossEntropy::CategoricalCrossEntropy(const std::string& reduction, bool from_logits,
                                                         float label_smoothing, const std::string& device)
            : reduction_(reduction), from_logits_(from_logits), label_smoothing_(label_smoothing), device_(device)
        {
            Layers::require_gpu_device(device_, "CategoricalCrossEntropy");
        }

        DeviceScalar CategoricalCrossEntropy::forward(const DeviceTensor& p, const DeviceTensor& t)
        {
            // categorical_cross_entropy.cpp:169-178
            if (!p.defined() || !t.defined() || p.size() == 0 || t.size() == 0)
                throw std::runtime_error("CategoricalCrossEntropy: Empty input tensors");
            if (p.rank() != 2 || p.dims() != t.dims())
                throw std::runtime_error("CategoricalCrossEntropy: Predictions and targets shape mismatch");
            const int red = cce_reduction(reduction_);
            const int64_t B = p.dimension(0), C = p.dimension(1);
            if (!probs_cache_.defined() || probs_cache_.dims() != p.dims())
            {
                probs_cache_ = DeviceTensor::empty(p.dims());
                targets_cache_ = DeviceTensor::empty(p.dims());
            }
            DeviceTensor loss = DeviceTensor::empty({1});
            Device::check(cnhip_cce_forward(p.data(), t.data(), probs_cache_.data(), targets_cache_.data(),
                                            loss.data(), B, C, from_logits_ ? 1 : 0, label_smoothing_,
                                            red, Device::stream()),
                          "CategoricalCrossEntropy::forward");
            return DeviceScalar(loss);
        }

        DeviceTensor CategoricalCrossEntropy::backward(const DeviceTensor& p, const DeviceTensor& t)
        {
            // categorical_cross_entropy.cpp:318-327
            if (!probs_cache_.defined())
                throw std::runtime_error("CategoricalCrossEntropy: Must call forward() before backward()");
            if (!p.defined() || !t.defined() || p.dims() != t.dims() || p.dims() != probs_cache_.dims())
                throw std::runtime_error("CategoricalCrossEntropy: Predictions and targets shape mismatch in backward");
            const int64_t B = p.dimension(0), C = p.dimension(1);
            DeviceTensor g = DeviceTensor::empty(p.dims());
            Device::check(cnhip_cce_backward(probs_cache_.data(), targets_cache_.data(), g.data(), B, C,
                                             from_logits_ ? 1 : 0, mean_or_sum(reduction_), Device::stream()),
                          "CategoricalCrossEntropy::backward");
            return g;
        }

        Tensor<float, 2> CategoricalCrossEntropy::one_hot(const std::vector<int>& labels, int64_t B, int64_t C) const
        {
            if (static_cast<int64_t>(labels.size()) != B)
                throw std::runtime_error(
                    "CategoricalCrossEntropy: Batch size mismatch between predictions and targets");
            Tensor<float, 2> oh(static_cast<int>(B), static_cast<int>(C));
            oh.setZero();
            for (int64_t b = 0; b < B; ++b)
            {
                const int c = labels[static_cast<size_t>(b)];
                if (c < 0 || c >= C) throw std::runtime_error("CategoricalCrossEntropy: Target index out of range");
                oh(static_cast<int>(b), c) = 1.0f;
            }
            return oh;
        }

        float CategoricalCrossEntropy::forward(const Tensor<float, 2>& p, const std::vector<int>& labels)
        {
            return Loss::forward(p, one_hot(labels, p.dimension(0), p.dimension(1)));
        }

        Tensor<float, 2> CategoricalCrossEntropy::backward(const Tensor<float, 2>& p, const std::vector<int>& labels)
        {
            return Loss::backward(p, one_hot(labels, p.dimension(0), p.dimension(1)));
        }

        // ---------------------------------------------------------------- MAE
        MAE::MAE(const std::string& reduction, const std::string& device) : reduction_(reduction), device_(device)
        {
            Layers::require_gpu_device(device_, "MAE");
        }

        DeviceScalar MAE::forward(const DeviceTensor& p, const DeviceTensor& t)
        {
            same_shape(p, t, "MAE");
            DeviceTensor loss = DeviceTensor::empty({1});
            Device::check(cnhip_mae_forward(p.data(), t.data(), loss.data(), p.size(), mean_or_sum(reduction_),
                                            Device::stream()),
                          "MAE::forward");
            return DeviceScalar(loss);
        }

        DeviceTensor MAE::backward(const DeviceTensor& p, const DeviceTensor& t)
        {
            same_shape(p, t, "MAE");
            DeviceTensor g = DeviceTensor::empty(p.dims());
            Device::check(cnhip_mae_backward(p.data(), t.data(), g.data(), p.size(), mean_or_sum(reduction_),
                                             Device::stream()),
                          "MAE::backward");
            return g;
        }

        // ---------------------------------------------------------------- Huber
        Huber::Huber(float delta, const std::string& reduction, const std::string& device)
            : delta_(delta), reduction_(reduction), device_(device)
        {
            Layers::require_gpu_device(device_, "Huber");
        }

        DeviceScalar Huber::forward(const DeviceTensor& p, const DeviceTensor& t)
        {
            same_shape(p, t, "Huber");
            DeviceTensor loss = DeviceTensor::empty({1});
            Device::check(cnhip_huber_forward(p.data(), t.data(), loss.data(), p.size(), delta_,
                                              mean_or_sum(reduction_), Device::stream()),
                          "Huber::forward");
            return DeviceScalar(loss);
        }

        DeviceTensor Huber::backward(const DeviceTensor& p, const DeviceTensor& t)
        {
            same_shape(p, t, "Huber");
            DeviceTensor g = DeviceTensor::empty(p.dims());
            Device::check(cnhip_huber_backward(p.data(), t.data(), g.data(), p.size(), delta_,
                                               mean_or_sum(reduction_), Device::stream()),
                          "Huber::backward");
            return g;
        }
    } // namespace Losses

    namespace Optimizers
    {
        // ---------------------------------------------------------------- device optimizers
        DeviceOptimizer::DeviceOptimizer(int kind, float hyper, float epsilon, const std::string& device,
                                         const char* name)
            : kind_(kind), hyper_(hyper), epsilon_(epsilon), device_(device), name_(name)
        {
            Layers::require_gpu_device(device_, name);
        }

        void DeviceOptimizer::update(float* weights, const float* gradients, int size, float learning_rate)
        {
            update(weights, gradients, static_cast<int64_t>(size), learning_rate);
        }

        void DeviceOptimizer::update(float* weights, const float* gradients, int64_t size, float learning_rate)
        {
            if (size <= 0) return;
            float* s = nullptr;
            auto it = states_.find(weights);
            if (it == states_.end())
            {
                if (!cnhip_is_device_pointer(weights) || !cnhip_is_device_pointer(gradients))
                    throw std::invalid_argument(std::string(name_) +
                                                "::update: parameters and gradients must be device memory in "
                                                "the gpu backend");
                // zero state at a key's first update (momentum.cpp:93-95, adagrad.cpp:95-97, mrs_prop.cpp:95-97)
                it = states_.emplace(weights, kind_ == CNHIP_OPT_SGD ? DeviceTensor() : DeviceTensor::zeros({size}))
                         .first;
            }
            if (kind_ != CNHIP_OPT_SGD)
            {
                if (it->second.size() != size)
                    throw std::invalid_argument(std::string(name_) + "::update: parameter size changed for a key");
                s = it->second.data();
            }
            pending_.push_back(Pending{weights, gradients, s, size, learning_rate});
            if (group_depth_ == 0) flush();
        }

        void DeviceOptimizer::begin_group() { ++group_depth_; }

        void DeviceOptimizer::end_group()
        {
            if (group_depth_ > 0 && --group_depth_ == 0) flush();
        }

        void DeviceOptimizer::flush()
        {
            size_t i = 0;
            while (i < pending_.size())
            {
                // one launch per run of equal learning rates (<= 64 tensors each)
                float* W[64];
                const float* G[64];
                float* S[64];
                int64_t N[64];
                const float lr = pending_[i].lr;
                int count = 0;
                while (i < pending_.size() && count < 64 && pending_[i].lr == lr)
                {
                    const Pending& p = pending_[i++];
                    W[count] = p.w; G[count] = p.g; S[count] = p.s; N[count] = p.n;
                    ++count;
                }
                const int st = cnhip_optimizer_step_multi(kind_, count, W, G, S, N, lr, hyper_, epsilon_,
                                                          Device::stream());
                if (st != CNHIP_OK)
                {
                    pending_.clear();
                    Device::check(st, name_);
                }
            }
            pending_.clear();
        }

        const DeviceTensor& DeviceOptimizer::state(const float* weights) const
        {
            auto it = states_.find(weights);
            if (it == states_.end()) throw std::out_of_range(std::string(name_) + ": no state for this parameter");
            return it->second;
        }

        int DeviceOptimizer::state_tensors() const { return kind_ == CNHIP_OPT_SGD ? 0 : 1; }

        bool DeviceOptimizer::get_state(const float* weights, int64_t n, std::vector<std::vector<float>>& tensors,
                                        int& t) const
        {
            auto it = states_.find(weights);
            if (it == states_.end()) return false;
            t = 0;
            tensors.clear();
            if (kind_ == CNHIP_OPT_SGD) return true;
            if (it->second.size() != n) throw std::invalid_argument(std::string(name_) + "::get_state: size mismatch");
            tensors.assign(1, std::vector<float>(static_cast<size_t>(n)));
            it->second.copy_to_host(tensors[0].data());
            return true;
        }

        void DeviceOptimizer::set_state(const float* weights, int64_t n,
                                        const std::vector<std::vector<float>>& tensors, int /*t*/)
        {
            const size_t want = static_cast<size_t>(state_tensors());
            if (tensors.size() != want || (want == 1 && static_cast<int64_t>(tensors[0].size()) != n))
                throw std::invalid_argument(std::string(name_) + "::set_state: state does not match the parameter");
            if (!cnhip_is_device_pointer(weights))
                throw std::invalid_argument(std::string(name_) + "::set_state: parameters must be device memory");
            auto it = states_.find(weights);
            if (it == states_.end())
                it = states_.emplace(weights, want ? DeviceTensor::empty({n}) : DeviceTensor()).first;
            if (want)
            {
                if (it->second.size() != n)
                    throw std::invalid_argument(std::string(name_) + "::set_state: size mismatch");
                it->second.copy_from_host(tensors[0].data());
            }
        }

        SGD::SGD(const std::string& device, int gpu_block_size)
            : DeviceOptimizer(CNHIP_OPT_SGD, 0.0f, 0.0f, device, "SGD"), block_(gpu_block_size)
        {
        }
        Momentum::Momentum(float mu, const std::string& device)
            : DeviceOptimizer(CNHIP_OPT_MOMENTUM, mu, 0.0f, device, "Momentum"), mu_(mu)
        {
        }
        Adagrad::Adagrad(float epsilon, const std::string& device)
            : DeviceOptimizer(CNHIP_OPT_ADAGRAD, 0.0f, epsilon, device, "Adagrad"), eps_(epsilon)
        {
        }
        RMSProp::RMSProp(float rho, float epsilon, const std::string& device)
            : DeviceOptimizer(CNHIP_OPT_RMSPROP, rho, epsilon, device, "RMSProp"), rho_(rho)
        {
        }
    } // namespace Optimizers

    namespace Layers
    {
        // ---------------------------------------------------------------- Dropout
        Dropout::Dropout(float p, const std::string& device) : p_(p), device_(device), seed_(Utils::next_seed())
        {
            if (p_ < 0.0f || p_ >= 1.0f) throw std::invalid_argument("Dropout probability must be in [0, 1)");
            require_gpu_device(device_, "Dropout");
        }

        DeviceTensor Dropout::forward(const DeviceTensor& x)
        {
            applied_ = training_ && p_ != 0.0f;  // dropout.cpp:143-144: identity otherwise
            if (!applied_) return x;
            DeviceTensor y = DeviceTensor::empty(x.dims());
            // one byte per element, held in a buffer of ceil(n / 4) words
            mask_n_ = x.size();
            mask_ = DeviceTensor::empty({(mask_n_ + 3) / 4});
            Device::check(cnhip_dropout_forward(x.data(), y.data(), reinterpret_cast<uint8_t*>(mask_.data()), x.size(), p_,
                                                seed_, offset_, Device::stream()),
                          "Dropout::forward");
            offset_ += static_cast<uint64_t>(x.size());
            return y;
        }

        DeviceTensor Dropout::backward(const DeviceTensor& g)
        {
            if (!training_ || p_ == 0.0f) return g;
            if (!applied_ || mask_n_ != g.size())
                throw std::runtime_error("Dropout::backward before a training forward of this shape");
            DeviceTensor dx = DeviceTensor::empty(g.dims());
            Device::check(cnhip_dropout_backward(g.data(), reinterpret_cast<const uint8_t*>(mask_.data()), dx.data(),
                                                 g.size(), p_, Device::stream()),
                          "Dropout::backward");
            return dx;
        }

        Tensor<float, 2> Dropout::forward(const Tensor<float, 2>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 2>();
        }
        Tensor<float, 4> Dropout::forward(const Tensor<float, 4>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 4>();
        }
        Tensor<float, 2> Dropout::backward(const Tensor<float, 2>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 2>();
        }
        Tensor<float, 4> Dropout::backward(const Tensor<float, 4>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 4>();
        }

        std::vector<float> Dropout::get_mask() const
        {
            if (!applied_) return {};
            std::vector<uint8_t> m(static_cast<size_t>(mask_.size()) * 4);
            mask_.copy_to_host(m.data());
            return std::vector<float>(m.begin(), m.begin() + mask_n_);
        }

        // ---------------------------------------------------------------- global pools
        static void check_4d(const DeviceTensor& x, const char* who)
        {
            if (x.rank() != 4 || x.size() == 0)
                throw std::runtime_error(std::string(who) + ": expected a non-empty [N, C, H, W] input, got " +
                                         shape_str(x.dims()));
        }

        GlobalAvgPool2D::GlobalAvgPool2D(const std::string& device) : device_(device)
        {
            require_gpu_device(device_, "GlobalAvgPool2D");
        }

        DeviceTensor GlobalAvgPool2D::forward(const DeviceTensor& x)
        {
            check_4d(x, "GlobalAvgPool2D::forward");
            in_dims_ = x.dims();
            DeviceTensor y = DeviceTensor::empty({in_dims_[0], in_dims_[1]});
            Device::check(cnhip_global_avgpool_forward(x.data(), y.data(), in_dims_[0], in_dims_[1], in_dims_[2],
                                                       in_dims_[3], Device::stream()),
                          "GlobalAvgPool2D::forward");
            return y;
        }

        DeviceTensor GlobalAvgPool2D::backward(const DeviceTensor& g)
        {
            if (in_dims_.empty()) throw std::runtime_error("GlobalAvgPool2D::backward before forward");
            if (g.rank() != 2 || g.dimension(0) != in_dims_[0] || g.dimension(1) != in_dims_[1])
                throw std::runtime_error("GlobalAvgPool2D::backward: grad shape " + shape_str(g.dims()));
            DeviceTensor dx = DeviceTensor::empty(in_dims_);
            Device::check(cnhip_global_avgpool_backward(g.data(), dx.data(), in_dims_[0], in_dims_[1], in_dims_[2],
                                                        in_dims_[3], Device::stream()),
                          "GlobalAvgPool2D::backward");
            return dx;
        }

        Tensor<float, 2> GlobalAvgPool2D::forward(const Tensor<float, 4>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 2>();
        }
        Tensor<float, 4> GlobalAvgPool2D::backward(const Tensor<float, 2>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 4>();
        }

        GlobalMaxPool2D::GlobalMaxPool2D(const std::string& device) : device_(device)
        {
            require_gpu_device(device_, "GlobalMaxPool2D");
        }

        DeviceTensor GlobalMaxPool2D::forward(const DeviceTensor& x)
        {
            check_4d(x, "GlobalMaxPool2D::forward");
            in_dims_ = x.dims();
            DeviceTensor y = DeviceTensor::empty({in_dims_[0], in_dims_[1]});
            ah_ = DeviceTensor::empty({in_dims_[0], in_dims_[1]});
            aw_ = DeviceTensor::empty({in_dims_[0], in_dims_[1]});
            Device::check(cnhip_global_maxpool_forward(x.data(), y.data(), ah_.idata(),
                                                       aw_.idata(), in_dims_[0], in_dims_[1],
                                                       in_dims_[2], in_dims_[3], Device::stream()),
                          "GlobalMaxPool2D::forward");
            return y;
        }

        DeviceTensor GlobalMaxPool2D::backward(const DeviceTensor& g)
        {
            if (in_dims_.empty()) throw std::runtime_error("GlobalMaxPool2D::backward before forward");
            if (g.rank() != 2 || g.dimension(0) != in_dims_[0] || g.dimension(1) != in_dims_[1])
                throw std::runtime_error("GlobalMaxPool2D::backward: grad shape " + shape_str(g.dims()));
            DeviceTensor dx = DeviceTensor::empty(in_dims_);
            Device::check(cnhip_global_maxpool_backward(g.data(), ah_.idata(),
                                                        aw_.idata(), dx.data(),
                                                        in_dims_[0], in_dims_[1], in_dims_[2], in_dims_[3],
                                                        Device::stream()),
                          "GlobalMaxPool2D::backward");
            return dx;
        }

        Tensor<float, 2> GlobalMaxPool2D::forward(const Tensor<float, 4>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 2>();
        }
        Tensor<float, 4> GlobalMaxPool2D::backward(const Tensor<float, 2>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 4>();
        }

        std::vector<int32_t> GlobalMaxPool2D::get_argmax_h() const
        {
            std::vector<int32_t> v(static_cast<size_t>(ah_.size()));
            if (!v.empty()) ah_.copy_to_host(v.data());
            return v;
        }
        std::vector<int32_t> GlobalMaxPool2D::get_argmax_w() const
        {
            std::vector<int32_t> v(static_cast<size_t>(aw_.size()));
            if (!v.empty()) aw_.copy_to_host(v.data());
            return v;
        }

        // ---------------------------------------------------------------- RNN
        RNN::RNN(int input_size, int hidden_size, bool return_sequences, const std::string& device)
            : RecurrentBase(input_size, hidden_size, return_sequences, 1, device, "RNN")
        {
        }

        DeviceTensor RNN::forward(const DeviceTensor& x)
        {
            check_input(x);
            const int64_t B = x.dimension(0), S = x.dimension(1);
            in_cache_ = x;
            out_cache_ = DeviceTensor::empty({B, S, static_cast<int64_t>(hidden_size_)});
            Device::check(cnhip_rnn_forward(x.data(), W_ih_.data(), W_hh_.data(), b_.data(), out_cache_.data(), B, S,
                                            input_size_, hidden_size_, Device::stream()),
                          "RNN::forward");
            return out_cache_;
        }

        DeviceTensor RNN::backward(const DeviceTensor& g) { return backward(g, true); }

        DeviceTensor RNN::backward(const DeviceTensor& g, bool input_grad)
        {
            if (!out_cache_.defined()) throw std::runtime_error("RNN::backward before forward");
            if (g.dims() != out_cache_.dims()) throw std::runtime_error("RNN::backward: grad shape mismatch");
            const int64_t B = g.dimension(0), S = g.dimension(1);
            DeviceTensor dx = input_grad ? DeviceTensor::empty(in_cache_.dims()) : DeviceTensor();
            Device::check(cnhip_rnn_backward(in_cache_.data(), W_ih_.data(), W_hh_.data(), out_cache_.data(), g.data(),
                                             gW_ih_.data(), gW_hh_.data(), gb_.data(), input_grad ? dx.data() : nullptr,
                                             B, S, input_size_, hidden_size_, Device::stream()),
                          "RNN::backward");
            grads_zero_ = false;
            return dx;
        }

        Tensor<float, 3> RNN::forward(const Tensor<float, 3>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 3>();
        }
        Tensor<float, 3> RNN::backward(const Tensor<float, 3>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 3>();
        }
    } // namespace Layers
} // namespace CppNet
