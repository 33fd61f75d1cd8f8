// LSTM / GRU on device "gpu" (ref: src/CppNet/layers/lstm.cpp:34-266,
// gru.cpp:30-322).
#include <cmath>
#include <stdexcept>
#include <string>
#include <vector>

#include "CppNet/layers/lstm.hpp"
#include "CppNet/optimizers/optimizer.hpp"
#include "CppNet/utils/init.hpp"

namespace CppNet
{
    namespace Layers
    {
        RecurrentBase::RecurrentBase(int input_size, int hidden_size, bool return_sequences, int gates,
                                     const std::string& device, const char* name)
            : input_size_(input_size), hidden_size_(hidden_size), gates_(gates),
              return_sequences_(return_sequences), device_(device), name_(name)
        {
            if (input_size <= 0 || hidden_size <= 0)
                throw std::invalid_argument(std::string(name) + ": sizes must be positive");
            require_gpu_device(device_, name);
            const int G = gates * hidden_size;
            // xavier-style limits (lstm.cpp:42-45, gru.cpp:36-39)
            const float lih = std::sqrt(6.0f / static_cast<float>(input_size + hidden_size));
            const float lhh = std::sqrt(6.0f / static_cast<float>(hidden_size + hidden_size));
            W_ih_ = DeviceTensor::empty({input_size, G});
            W_hh_ = DeviceTensor::empty({hidden_size, G});
            W_ih_.copy_from_host(Utils::uniform_init(input_size, G, -lih, lih).data());
            W_hh_.copy_from_host(Utils::uniform_init(hidden_size, G, -lhh, lhh).data());
            b_ = DeviceTensor::zeros({G});
            gW_ih_ = DeviceTensor::empty({input_size, G});
            gW_hh_ = DeviceTensor::empty({hidden_size, G});
            gb_ = DeviceTensor::empty({G});
        }

        void RecurrentBase::check_input(const DeviceTensor& x) const
        {
            if (x.rank() != 3 || x.dimension(2) != input_size_)
                throw std::runtime_error(std::string(name_) + "::forward: expected [B, S, " +
                                         std::to_string(input_size_) + "], got " + shape_str(x.dims()));
        }

        void RecurrentBase::materialize_grads() const
        {
            if (!grads_zero_) return;
            auto* self = const_cast<RecurrentBase*>(this);
            self->gW_ih_.fill_zero();
            self->gW_hh_.fill_zero();
            self->gb_.fill_zero();
            self->grads_zero_ = false;
        }

        void RecurrentBase::step(Optimizers::Optimizer& optimizer, float learning_rate)
        {
            if (!trainable_) return;
            materialize_grads();
            optimizer.update(W_ih_.data(), gW_ih_.data(), W_ih_.size(), learning_rate);
            optimizer.update(W_hh_.data(), gW_hh_.data(), W_hh_.size(), learning_rate);
            optimizer.update(b_.data(), gb_.data(), b_.size(), learning_rate);
            grads_zero_ = true;  // lstm.cpp:263-265 / gru.cpp:306-308 clear after the update
        }

        static void check_shape2(const Tensor<float, 2>& w, const DeviceTensor& d, const char* who)
        {
            if (w.dimension(0) != d.dimension(0) || w.dimension(1) != d.dimension(1))
                throw std::invalid_argument(std::string(who) + ": shape mismatch");
        }
        void RecurrentBase::set_W_ih(const Tensor<float, 2>& w)
        {
            check_shape2(w, W_ih_, "set_W_ih");
            W_ih_.copy_from_host(w.data());
        }
        void RecurrentBase::set_W_hh(const Tensor<float, 2>& w)
        {
            check_shape2(w, W_hh_, "set_W_hh");
            W_hh_.copy_from_host(w.data());
        }
        void RecurrentBase::set_bias(const Tensor<float, 1>& b)
        {
            if (b.dimension(0) != b_.dimension(0)) throw std::invalid_argument("set_bias: shape mismatch");
            b_.copy_from_host(b.data());
        }

        // ---------------------------------------------------------------- LSTM
        LSTM::LSTM(int input_size, int hidden_size, bool return_sequences, const std::string& device)
            : RecurrentBase(input_size, hidden_size, return_sequences, 4, device, "LSTM")
        {
            // forget-gate bias block = 1 (lstm.cpp:47-49)
            std::vector<float> b(static_cast<size_t>(4 * hidden_size), 0.0f);
            for (int d = hidden_size; d < 2 * hidden_size; ++d) b[static_cast<size_t>(d)] = 1.0f;
            b_.copy_from_host(b.data());
        }

        DeviceTensor LSTM::forward(const DeviceTensor& x)
        {
            check_input(x);
            const int64_t B = x.dimension(0), S = x.dimension(1), H = hidden_size_;
            in_cache_ = x;
            out_cache_ = DeviceTensor::empty({B, S, H});
            gates_cache_ = DeviceTensor::empty({B * S, 4 * H});
            c_cache_ = DeviceTensor::empty({B * S, H});
            tanh_c_cache_ = DeviceTensor::empty({B * S, H});
            Device::check(cnhip_lstm_forward(x.data(), W_ih_.data(), W_hh_.data(), b_.data(),
                                             out_cache_.data(), gates_cache_.data(), c_cache_.data(),
                                             tanh_c_cache_.data(), B, S, input_size_, H, Device::stream()),
                          "LSTM::forward");
            return out_cache_;
        }

        DeviceTensor LSTM::backward(const DeviceTensor& g) { return backward(g, true); }

        DeviceTensor LSTM::backward(const DeviceTensor& g, bool input_grad)
        {
            if (!out_cache_.defined()) throw std::runtime_error("LSTM::backward before forward");
            if (g.dims() != out_cache_.dims()) throw std::runtime_error("LSTM::backward: grad shape mismatch");
            const int64_t B = g.dimension(0), S = g.dimension(1);
            DeviceTensor dx = input_grad ? DeviceTensor::empty(in_cache_.dims()) : DeviceTensor();
            Device::check(cnhip_lstm_backward(in_cache_.data(), W_ih_.data(), W_hh_.data(), out_cache_.data(),
                                              gates_cache_.data(), c_cache_.data(), tanh_c_cache_.data(),
                                              g.data(), gW_ih_.data(), gW_hh_.data(), gb_.data(), input_grad ? dx.data() : nullptr,
                                              B, S, input_size_, hidden_size_, Device::stream()),
                          "LSTM::backward");
            grads_zero_ = false;
            return dx;
        }

        DeviceTensor LSTM::backward_last(const DeviceTensor& g, bool input_grad)
        {
            if (!out_cache_.defined()) throw std::runtime_error("LSTM::backward before forward");
            const int64_t B = out_cache_.dimension(0), S = out_cache_.dimension(1);
            if (g.rank() != 2 || g.dimension(0) != B || g.dimension(1) != hidden_size_)
                throw std::runtime_error("LSTM::backward_last: grad shape mismatch");
            DeviceTensor dx = input_grad ? DeviceTensor::empty(in_cache_.dims()) : DeviceTensor();
            Device::check(cnhip_lstm_backward_last(in_cache_.data(), W_ih_.data(), W_hh_.data(), out_cache_.data(),
                                                   gates_cache_.data(), c_cache_.data(), tanh_c_cache_.data(),
                                                   g.data(), gW_ih_.data(), gW_hh_.data(), gb_.data(),
                                                   input_grad ? dx.data() : nullptr, B, S, input_size_, hidden_size_,
                                                   Device::stream()),
                          "LSTM::backward_last");
            grads_zero_ = false;
            return dx;
        }

        Tensor<float, 3> LSTM::forward(const Tensor<float, 3>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 3>();
        }
        Tensor<float, 3> LSTM::backward(const Tensor<float, 3>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 3>();
        }

        // ---------------------------------------------------------------- GRU
        GRU::GRU(int input_size, int hidden_size, bool return_sequences, const std::string& device)
            : RecurrentBase(input_size, hidden_size, return_sequences, 3, device, "GRU")
        {
        }

        DeviceTensor GRU::forward(const DeviceTensor& x)
        {
            check_input(x);
            const int64_t B = x.dimension(0), S = x.dimension(1), H = hidden_size_;
            in_cache_ = x;
            out_cache_ = DeviceTensor::empty({B, S, H});
            gates_cache_ = DeviceTensor::empty({B * S, 3 * H});
            rh_cache_ = DeviceTensor::empty({B * S, H});
            Device::check(cnhip_gru_forward(x.data(), W_ih_.data(), W_hh_.data(), b_.data(),
                                            out_cache_.data(), gates_cache_.data(), rh_cache_.data(), B, S,
                                            input_size_, H, Device::stream()),
                          "GRU::forward");
            return out_cache_;
        }

        DeviceTensor GRU::backward(const DeviceTensor& g) { return backward(g, true); }

        DeviceTensor GRU::backward(const DeviceTensor& g, bool input_grad)
        {
            if (!out_cache_.defined()) throw std::runtime_error("GRU::backward before forward");
            if (g.dims() != out_cache_.dims()) throw std::runtime_error("GRU::backward: grad shape mismatch");
            const int64_t B = g.dimension(0), S = g.dimension(1);
            DeviceTensor dx = input_grad ? DeviceTensor::empty(in_cache_.dims()) : DeviceTensor();
            Device::check(cnhip_gru_backward(in_cache_.data(), W_ih_.data(), W_hh_.data(), out_cache_.data(),
                                             gates_cache_.data(), rh_cache_.data(), g.data(), gW_ih_.data(),
                                             gW_hh_.data(), gb_.data(), input_grad ? dx.data() : nullptr, B, S, input_size_,
                                             hidden_size_, Device::stream()),
                          "GRU::backward");
            grads_zero_ = false;
            return dx;
        }

        Tensor<float, 3> GRU::forward(const Tensor<float, 3>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 3>();
        }
        Tensor<float, 3> GRU::backward(const Tensor<float, 3>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 3>();
        }
    } // namespace Layers
} // namespace CppNet

#include "CppNet/layers/sequence_last.hpp"

namespace CppNet
{
    namespace Layers
    {
        DeviceTensor SequenceLast::forward(const DeviceTensor& x)
        {
            if (x.rank() != 3) throw std::runtime_error("SequenceLast: expected [B, S, D]");
            in_dims_ = x.dims();
            const int64_t B = x.dimension(0), S = x.dimension(1), D = x.dimension(2);
            DeviceTensor out = DeviceTensor::empty({B, D});
            Device::check(cnhip_seq_select(x.data(), out.data(), B, S, D, S - 1, Device::stream()),
                          "SequenceLast::forward");
            return out;
        }

        DeviceTensor SequenceLast::backward(const DeviceTensor& g)
        {
            if (in_dims_.size() != 3) throw std::runtime_error("SequenceLast::backward before forward");
            const int64_t B = in_dims_[0], S = in_dims_[1], D = in_dims_[2];
            DeviceTensor dx = DeviceTensor::empty(in_dims_);
            Device::check(cnhip_seq_scatter(g.data(), dx.data(), B, S, D, S - 1, Device::stream()),
                          "SequenceLast::backward");
            return dx;
        }
    } // namespace Layers
} // namespace CppNet
