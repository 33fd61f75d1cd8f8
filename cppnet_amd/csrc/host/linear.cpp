// Linear layer on device "gpu" (ref: src/CppNet/layers/linear.cpp).
#include "CppNet/layers/linear.hpp"

#include <iostream>
#include <stdexcept>

#include "CppNet/layers/max_pool2d.hpp"
#include "CppNet/optimizers/optimizer.hpp"
#include "CppNet/utils/init.hpp"

namespace CppNet
{
    namespace Layers
    {
        void require_gpu_device(const std::string& device, const std::string& who)
        {
            if (device != "gpu")
                throw std::runtime_error("Unknown device: " + device + " (" + who +
                                         "; this backend implements device \"gpu\")");
        }

        Linear::Linear(int in_size, int out_size, std::string layer_name, bool trainable, bool bias,
                       std::string device, std::string weight_init)
            : in_size_(in_size), out_size_(out_size), layer_name_(std::move(layer_name)),
              trainable_(trainable), bias_flag_(bias), device_(std::move(device)),
              weight_init_(std::move(weight_init))
        {
            if (in_size <= 0 || out_size <= 0)
                throw std::invalid_argument("Linear: sizes must be positive in layer: " + layer_name_);
            require_gpu_device(device_, "Linear " + layer_name_);
            W_ = DeviceTensor::empty({in_size_, out_size_});
            gW_ = DeviceTensor::empty({in_size_, out_size_});  // zero by grads_zero_
            set_weights(Utils::init_weights(in_size_, out_size_, weight_init_));
            if (bias_flag_)
            {
                b_ = DeviceTensor::zeros({out_size_});   // biases start at zero (linear.cpp:75-80)
                gb_ = DeviceTensor::empty({out_size_});
            }
        }

        DeviceTensor Linear::forward(const DeviceTensor& input)
        {
            if (input.rank() != 2 || input.dimension(1) != in_size_)
                throw std::runtime_error("Shape mismatch: in layer: " + layer_name_ +
                                         " input.dimension(1) must be equal weights_.dimension(0)!");
            in_cache_ = input;
            const int64_t B = input.dimension(0);
            DeviceTensor out = DeviceTensor::empty({B, out_size_});
            Device::check(cnhip_linear_forward(input.data(), W_.data(),
                                               bias_flag_ ? b_.data() : nullptr, out.data(), B,
                                               in_size_, out_size_, Device::stream()),
                          "Linear::forward");
            return out;
        }

        DeviceTensor Linear::forward_act(const DeviceTensor& input, int act, DeviceTensor* pre_act)
        {
            if (input.rank() != 2 || input.dimension(1) != in_size_)
                throw std::runtime_error("Shape mismatch: in layer: " + layer_name_ +
                                         " input.dimension(1) must be equal weights_.dimension(0)!");
            if (act == CNHIP_ACT_GELU && !pre_act)
                throw std::invalid_argument("Linear::forward_act: GELU needs the pre-activation output");
            in_cache_ = input;
            const int64_t B = input.dimension(0);
            DeviceTensor out = DeviceTensor::empty({B, out_size_});
            DeviceTensor z;
            if (act == CNHIP_ACT_GELU) z = DeviceTensor::empty({B, out_size_});
            Device::check(cnhip_linear_forward_act(input.data(), W_.data(), bias_flag_ ? b_.data() : nullptr,
                                                   out.data(), z.defined() ? z.data() : nullptr, B, in_size_,
                                                   out_size_, act, Device::stream()),
                          "Linear::forward_act");
            if (pre_act) *pre_act = z;
            return out;
        }

        DeviceTensor Linear::forward_residual(const DeviceTensor& input, const DeviceTensor& residual)
        {
            if (input.rank() != 2 || input.dimension(1) != in_size_)
                throw std::runtime_error("Shape mismatch: in layer: " + layer_name_ +
                                         " input.dimension(1) must be equal weights_.dimension(0)!");
            const int64_t B = input.dimension(0);
            if (residual.size() != B * out_size_)
                throw std::runtime_error("Linear::forward_residual: residual does not match the output in layer: " +
                                         layer_name_);
            in_cache_ = input;
            DeviceTensor out = DeviceTensor::empty({B, out_size_});
            Device::check(cnhip_linear_forward_act(input.data(), W_.data(), bias_flag_ ? b_.data() : nullptr,
                                                   out.data(), const_cast<float*>(residual.data()), B, in_size_,
                                                   out_size_, CNHIP_ACT_RESIDUAL, Device::stream()),
                          "Linear::forward_residual");
            return out;
        }

        DeviceTensor Linear::backward_act(const DeviceTensor& grad_output, int act, const DeviceTensor& act_aux)
        {
            if (grad_output.rank() != 2 || grad_output.dimension(1) != out_size_)
                throw std::runtime_error("Output size mismatch in layer: " + layer_name_);
            if (!in_cache_.defined() || in_cache_.dimension(0) != grad_output.dimension(0))
                throw std::runtime_error("Linear::backward before forward (or batch mismatch) in layer: " +
                                         layer_name_);
            const int64_t B = grad_output.dimension(0);
            if (act != CNHIP_ACT_NONE && act_aux.size() != B * in_size_)
                throw std::runtime_error("Linear::backward_act: activation tensor does not match the input");
            DeviceTensor dX = DeviceTensor::empty({B, in_size_});
            const int accumulate = grads_zero_ ? 0 : 1;
            Device::check(cnhip_linear_backward_act(in_cache_.data(), W_.data(), grad_output.data(), gW_.data(),
                                                    bias_flag_ ? gb_.data() : nullptr, dX.data(),
                                                    act == CNHIP_ACT_NONE ? nullptr : act_aux.data(), B,
                                                    in_size_, out_size_, trainable_ ? 1 : 0, accumulate, act,
                                                    Device::stream()),
                          "Linear::backward_act");
            if (trainable_) grads_zero_ = false;
            return dX;
        }

        DeviceTensor Linear::backward(const DeviceTensor& grad_output) { return backward(grad_output, true); }

        DeviceTensor Linear::backward(const DeviceTensor& grad_output, bool input_grad)
        {
            if (grad_output.rank() != 2 || grad_output.dimension(1) != out_size_)
                throw std::runtime_error("Output size mismatch in layer: " + layer_name_);
            if (!in_cache_.defined() || in_cache_.dimension(0) != grad_output.dimension(0))
                throw std::runtime_error("Linear::backward before forward (or batch mismatch) in layer: " +
                                         layer_name_);
            const int64_t B = grad_output.dimension(0);
            DeviceTensor dX = input_grad ? DeviceTensor::empty({B, in_size_}) : DeviceTensor();
            // grad_W += X^T dY (linear.cpp:346-352); over known-zero grads, write.
            const int accumulate = grads_zero_ ? 0 : 1;
            Device::check(cnhip_linear_backward(in_cache_.data(), W_.data(), grad_output.data(),
                                                gW_.data(), bias_flag_ ? gb_.data() : nullptr,
                                                input_grad ? dX.data() : nullptr, B, in_size_, out_size_, trainable_ ? 1 : 0,
                                                accumulate, Device::stream()),
                          "Linear::backward");
            if (trainable_) grads_zero_ = false;
            return dX;
        }

        bool Linear::fuses_maxpool_backward(const DeviceTensor& g, const MaxPool2D& pool) const
        {
            if (!trainable_ || !pool.fused_forward() || !in_cache_.defined()) return false;
            const DeviceTensor& P = pool.pooled_output();
            const std::vector<int64_t>& d = pool.input_dims();
            if (in_cache_.data() != P.data() || in_cache_.size() != P.size() || d.size() != 4) return false;
            if (g.rank() != 2 || g.dimension(0) != d[0] || g.dimension(1) != out_size_) return false;
            return cnhip_linear_backward_maxpool_relu_fits(d[0], d[1], d[2], d[3], out_size_, pool.get_pool_size(),
                                                           pool.get_stride()) != 0;
        }

        DeviceTensor Linear::backward_maxpool_relu(const DeviceTensor& g, const MaxPool2D& pool)
        {
            if (!fuses_maxpool_backward(g, pool))
                throw std::runtime_error("Linear::backward_maxpool_relu: the input is not the pooled output of a "
                                         "fused Conv2D -> ReLU -> MaxPool2D forward, or the shapes do not fit, "
                                         "in layer: " + layer_name_);
            const std::vector<int64_t>& d = pool.input_dims();
            DeviceTensor dx = DeviceTensor::empty(d);
            const int accumulate = grads_zero_ ? 0 : 1;
            Device::check(cnhip_linear_backward_maxpool_relu(in_cache_.data(), pool.max_indices().idata(), W_.data(),
                                                             g.data(), gW_.data(), bias_flag_ ? gb_.data() : nullptr,
                                                             dx.data(), d[0], d[1], d[2], d[3], out_size_,
                                                             pool.get_pool_size(), pool.get_stride(), accumulate,
                                                             Device::stream()),
                          "Linear::backward_maxpool_relu");
            grads_zero_ = false;
            return dx;
        }

        Tensor<float, 2> Linear::forward(const Tensor<float, 2>& input)
        {
            return forward(DeviceTensor::from_host(input)).to_host<float, 2>();
        }

        Tensor<float, 2> Linear::backward(const Tensor<float, 2>& grad_output)
        {
            return backward(DeviceTensor::from_host(grad_output)).to_host<float, 2>();
        }

        void Linear::materialize_grads() const
        {
            if (!grads_zero_) return;
            auto* self = const_cast<Linear*>(this);
            self->gW_.fill_zero();
            if (bias_flag_) self->gb_.fill_zero();
            self->grads_zero_ = false;
        }

        void Linear::step(Optimizers::Optimizer& optimizer, float learning_rate)
        {
            if (!trainable_) return;
            materialize_grads();
            optimizer.update(W_.data(), gW_.data(), W_.size(), learning_rate);
            if (bias_flag_) optimizer.update(b_.data(), gb_.data(), b_.size(), learning_rate);
        }

        void Linear::reset_grads()
        {
            if (!trainable_) return;
            grads_zero_ = true;
        }

        const Tensor<float, 2> Linear::get_weights() const { return W_.to_host<float, 2>(); }
        const Tensor<float, 2> Linear::get_grad_weights() const
        {
            materialize_grads();
            return gW_.to_host<float, 2>();
        }
        const Tensor<float, 1> Linear::get_biases() const
        {
            return bias_flag_ ? b_.to_host<float, 1>() : Tensor<float, 1>(0);
        }
        const Tensor<float, 1> Linear::get_grad_biases() const
        {
            materialize_grads();
            return bias_flag_ ? gb_.to_host<float, 1>() : Tensor<float, 1>(0);
        }

        void Linear::set_weights(const Tensor<float, 2>& w)
        {
            if (w.dimension(0) != in_size_ || w.dimension(1) != out_size_)
                throw std::invalid_argument("Linear::set_weights: shape mismatch in layer: " + layer_name_);
            W_.copy_from_host(w.data());
        }

        void Linear::set_biases(const Tensor<float, 1>& b)
        {
            if (!bias_flag_) throw std::invalid_argument("Linear::set_biases: layer has no bias: " + layer_name_);
            if (b.dimension(0) != out_size_)
                throw std::invalid_argument("Linear::set_biases: shape mismatch in layer: " + layer_name_);
            b_.copy_from_host(b.data());
        }

        void Linear::reinitialize_weights(const std::string& method)
        {
            set_weights(Utils::init_weights(in_size_, out_size_, method));
            weight_init_ = method;
            if (bias_flag_) b_.fill_zero();
        }

        void Linear::set_max_batch_size(int max_batch_size)
        {
            if (max_batch_size <= 0)
                throw std::invalid_argument("Linear::set_max_batch_size: must be positive");
        }

        void Linear::print_layer_info() const
        {
            std::cout << "Linear " << layer_name_ << ": " << in_size_ << " -> " << out_size_
                      << (bias_flag_ ? " (bias)" : "") << " device=" << device_
                      << (trainable_ ? "" : " [frozen]") << "\n";
        }
    } // namespace Layers
} // namespace CppNet
