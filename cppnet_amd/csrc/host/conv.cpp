// Conv2D / MaxPool2D / Flatten on device "gpu" (ref: src/CppNet/layers/
// conv2d.cpp:29-213, max_pool2d.cpp:25-131, flatten.cpp:15-39).
#include <cmath>
#include <random>
#include <stdexcept>
#include <string>

#include "CppNet/layers/conv2d.hpp"
#include "CppNet/layers/flatten.hpp"
#include "CppNet/layers/max_pool2d.hpp"
#include "CppNet/optimizers/optimizer.hpp"
#include "CppNet/utils/init.hpp"

namespace CppNet
{
    namespace Layers
    {
        // ---------------------------------------------------------------- Conv2D
        Conv2D::Conv2D(int in_channels, int out_channels, int kernel_size, int stride, int padding,
                       bool bias, const std::string& device)
            : in_channels_(in_channels), out_channels_(out_channels), kernel_size_(kernel_size),
              stride_(stride), padding_(padding), bias_flag_(bias), device_(device)
        {
            if (in_channels <= 0 || out_channels <= 0 || kernel_size <= 0 || stride <= 0 || padding < 0)
                throw std::invalid_argument("Conv2D: invalid configuration");
            require_gpu_device(device_, "Conv2D");
            const int64_t ks = kernel_size_;
            W_ = DeviceTensor::empty({out_channels_, in_channels_, ks, ks});
            gW_ = DeviceTensor::empty({out_channels_, in_channels_, ks, ks});
            // xavier-uniform over fan_in = C*k^2, fan_out = OC*k^2, drawn as a
            // [OC, C*k*k] matrix and reinterpreted (conv2d.cpp:42-50)
            const float fan_in = static_cast<float>(in_channels_ * kernel_size_ * kernel_size_);
            const float fan_out = static_cast<float>(out_channels_ * kernel_size_ * kernel_size_);
            const float limit = std::sqrt(6.0f / (fan_in + fan_out));
            auto w = Utils::uniform_init(out_channels_, in_channels_ * kernel_size_ * kernel_size_, -limit, limit);
            W_.copy_from_host(w.data());
            if (bias_flag_)
            {
                b_ = DeviceTensor::zeros({out_channels_});
                gb_ = DeviceTensor::empty({out_channels_});
            }
        }

        DeviceTensor Conv2D::forward(const DeviceTensor& x) { return forward_impl(x, false); }
        DeviceTensor Conv2D::forward_relu(const DeviceTensor& x) { return forward_impl(x, true); }

        DeviceTensor Conv2D::forward_impl(const DeviceTensor& x, bool relu)
        {
            if (x.rank() != 4 || x.dimension(1) != in_channels_)
                throw std::runtime_error("Conv2D::forward: expected [N, " + std::to_string(in_channels_) +
                                         ", H, W], got " + shape_str(x.dims()));
            in_cache_ = x;
            const int64_t N = x.dimension(0), H = x.dimension(2), W = x.dimension(3);
            const int64_t HO = (H + 2 * padding_ - kernel_size_) / stride_ + 1;
            const int64_t WO = (W + 2 * padding_ - kernel_size_) / stride_ + 1;
            if (HO <= 0 || WO <= 0) throw std::runtime_error("Conv2D::forward: input smaller than kernel");
            DeviceTensor y = DeviceTensor::empty({N, out_channels_, HO, WO});
            const auto fwd = relu ? cnhip_conv2d_forward_relu : cnhip_conv2d_forward;
            Device::check(fwd(x.data(), W_.data(), bias_flag_ ? b_.data() : nullptr, y.data(), N,
                              in_channels_, H, W, out_channels_, kernel_size_, stride_, padding_,
                              Device::stream()),
                          relu ? "Conv2D::forward_relu" : "Conv2D::forward");
            return y;
        }

        DeviceTensor Conv2D::forward_relu_maxpool(const DeviceTensor& x, MaxPool2D& pool)
        {
            if (x.rank() != 4 || x.dimension(1) != in_channels_)
                throw std::runtime_error("Conv2D::forward: expected [N, " + std::to_string(in_channels_) +
                                         ", H, W], got " + shape_str(x.dims()));
            const int64_t N = x.dimension(0), H = x.dimension(2), W = x.dimension(3);
            const int64_t HO = (H + 2 * padding_ - kernel_size_) / stride_ + 1;
            const int64_t WO = (W + 2 * padding_ - kernel_size_) / stride_ + 1;
            if (HO <= 0 || WO <= 0) throw std::runtime_error("Conv2D::forward: input smaller than kernel");
            const int64_t ps = pool.get_pool_size(), pst = pool.get_stride();
            if (HO < ps || WO < ps) throw std::runtime_error("MaxPool2D::forward: input smaller than the pool window");
            const int64_t HP = (HO - ps) / pst + 1, WP = (WO - ps) / pst + 1;
            in_cache_ = x;
            DeviceTensor y = DeviceTensor::empty({N, out_channels_, HP, WP});
            DeviceTensor idx = DeviceTensor::empty({N, out_channels_, HP, WP});  // int32 payload
            Device::check(cnhip_conv2d_forward_relu_maxpool(x.data(), W_.data(), bias_flag_ ? b_.data() : nullptr,
                                                            y.data(), idx.idata(), N, in_channels_, H, W,
                                                            out_channels_, kernel_size_, stride_, padding_, ps,
                                                            pst, Device::stream()),
                          "Conv2D::forward_relu_maxpool");
            pool.set_fused_forward({N, out_channels_, HO, WO}, y, idx);
            return y;
        }

        DeviceTensor Conv2D::backward(const DeviceTensor& g) { return backward(g, true); }

        DeviceTensor Conv2D::backward(const DeviceTensor& g, bool input_grad)
        {
            if (!in_cache_.defined()) throw std::runtime_error("Conv2D::backward before forward");
            const int64_t N = in_cache_.dimension(0), H = in_cache_.dimension(2), W = in_cache_.dimension(3);
            DeviceTensor dx = input_grad ? DeviceTensor::empty(in_cache_.dims()) : DeviceTensor();
            Device::check(cnhip_conv2d_backward(in_cache_.data(), W_.data(), g.data(), gW_.data(),
                                                bias_flag_ ? gb_.data() : nullptr,
                                                input_grad ? dx.data() : nullptr, N,
                                                in_channels_, H, W, out_channels_, kernel_size_, stride_,
                                                padding_, Device::stream()),
                          "Conv2D::backward");
            grads_zero_ = false;
            return dx;
        }

        bool Conv2D::fuses_pool_backward(const DeviceTensor& g, const MaxPool2D& pool) const
        {
            if (!trainable_ || !in_cache_.defined() || !pool.fused_forward()) return false;
            const std::vector<int64_t>& d = pool.input_dims();
            const int64_t N = in_cache_.dimension(0), H = in_cache_.dimension(2), W = in_cache_.dimension(3);
            if (d.size() != 4 || d[0] != N || d[1] != out_channels_ || g.size() != pool.pooled_output().size())
                return false;
            return cnhip_conv2d_backward_maxpool_relu_fits(N, in_channels_, H, W, out_channels_, kernel_size_,
                                                           stride_, padding_, pool.get_pool_size(),
                                                           pool.get_stride()) != 0;
        }

        void Conv2D::backward_params_maxpool_relu(const DeviceTensor& g, const MaxPool2D& pool)
        {
            if (!fuses_pool_backward(g, pool))
                throw std::runtime_error("Conv2D::backward_params_maxpool_relu: the pool's forward was not fused "
                                         "into this layer's, or the shape does not fit");
            const int64_t N = in_cache_.dimension(0), H = in_cache_.dimension(2), W = in_cache_.dimension(3);
            Device::check(cnhip_conv2d_backward_maxpool_relu(in_cache_.data(), g.data(), pool.max_indices().idata(),
                                                             pool.pooled_output().data(), gW_.data(),
                                                             bias_flag_ ? gb_.data() : nullptr, N, in_channels_, H,
                                                             W, out_channels_, kernel_size_, stride_, padding_,
                                                             pool.get_pool_size(), pool.get_stride(),
                                                             Device::stream()),
                          "Conv2D::backward_params_maxpool_relu");
            grads_zero_ = false;
        }

        Tensor<float, 4> Conv2D::forward(const Tensor<float, 4>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 4>();
        }
        Tensor<float, 4> Conv2D::backward(const Tensor<float, 4>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 4>();
        }

        void Conv2D::materialize_grads() const
        {
            if (!grads_zero_) return;
            auto* self = const_cast<Conv2D*>(this);
            self->gW_.fill_zero();
            if (bias_flag_) self->gb_.fill_zero();
            self->grads_zero_ = false;
        }

        void Conv2D::step(Optimizers::Optimizer& optimizer, float learning_rate)
        {
            if (!trainable_) return;
            materialize_grads();
            optimizer.update(W_.data(), gW_.data(), W_.size(), learning_rate);
            if (bias_flag_) optimizer.update(b_.data(), gb_.data(), b_.size(), learning_rate);
            grads_zero_ = true;  // conv2d.cpp:211-212 clears the grads after the update
        }

        const Tensor<float, 4> Conv2D::get_weights() const { return W_.to_host<float, 4>(); }
        const Tensor<float, 1> Conv2D::get_biases() const
        {
            return bias_flag_ ? b_.to_host<float, 1>() : Tensor<float, 1>(0);
        }
        const Tensor<float, 4> Conv2D::get_grad_weights() const
        {
            materialize_grads();
            return gW_.to_host<float, 4>();
        }
        const Tensor<float, 1> Conv2D::get_grad_biases() const
        {
            materialize_grads();
            return bias_flag_ ? gb_.to_host<float, 1>() : Tensor<float, 1>(0);
        }
        void Conv2D::set_weights(const Tensor<float, 4>& w)
        {
            for (int i = 0; i < 4; ++i)
                if (w.dimension(i) != W_.dimension(i))
                    throw std::invalid_argument("Conv2D::set_weights: shape mismatch");
            W_.copy_from_host(w.data());
        }
        void Conv2D::set_biases(const Tensor<float, 1>& b)
        {
            if (!bias_flag_ || b.dimension(0) != out_channels_)
                throw std::invalid_argument("Conv2D::set_biases: shape mismatch or no bias");
            b_.copy_from_host(b.data());
        }

        // ---------------------------------------------------------------- MaxPool2D
        MaxPool2D::MaxPool2D(int pool_size, int stride, const std::string& device)
            : pool_size_(pool_size), stride_(stride > 0 ? stride : pool_size), device_(device)
        {
            if (pool_size <= 0) throw std::invalid_argument("MaxPool2D: pool_size must be positive");
            require_gpu_device(device_, "MaxPool2D");
        }

        DeviceTensor MaxPool2D::forward(const DeviceTensor& x)
        {
            if (x.rank() != 4) throw std::runtime_error("MaxPool2D::forward: expected a 4-D input");
            const int64_t N = x.dimension(0), C = x.dimension(1), H = x.dimension(2), W = x.dimension(3);
            if (H < pool_size_ || W < pool_size_)
                throw std::runtime_error("MaxPool2D::forward: input smaller than the pool window");
            const int64_t HO = (H - pool_size_) / stride_ + 1, WO = (W - pool_size_) / stride_ + 1;
            in_dims_ = x.dims();
            fused_out_ = DeviceTensor();
            DeviceTensor y = DeviceTensor::empty({N, C, HO, WO});
            idx_ = DeviceTensor::empty({N, C, HO, WO});  // int32 payload
            Device::check(cnhip_maxpool2d_forward(x.data(), y.data(), idx_.idata(), N, C, H, W, pool_size_,
                                                  stride_, Device::stream()),
                          "MaxPool2D::forward");
            return y;
        }

        DeviceTensor MaxPool2D::backward(const DeviceTensor& g)
        {
            if (!idx_.defined()) throw std::runtime_error("MaxPool2D::backward before forward");
            if (g.size() != idx_.size()) throw std::runtime_error("MaxPool2D::backward: grad shape mismatch");
            DeviceTensor dx = DeviceTensor::empty(in_dims_);
            Device::check(cnhip_maxpool2d_backward(g.data(), idx_.idata(), dx.data(), in_dims_[0],
                                                   in_dims_[1], in_dims_[2], in_dims_[3], pool_size_,
                                                   stride_, Device::stream()),
                          "MaxPool2D::backward");
            return dx;
        }

        DeviceTensor MaxPool2D::backward_relu(const DeviceTensor& g, const DeviceTensor& relu_out)
        {
            if (!idx_.defined()) throw std::runtime_error("MaxPool2D::backward before forward");
            if (g.size() != idx_.size()) throw std::runtime_error("MaxPool2D::backward: grad shape mismatch");
            if (relu_out.dims() != in_dims_)
                throw std::runtime_error("MaxPool2D::backward_relu: ReLU output does not match the input");
            DeviceTensor dx = DeviceTensor::empty(in_dims_);
            Device::check(cnhip_maxpool2d_backward_relu(g.data(), idx_.idata(), relu_out.data(), dx.data(),
                                                        in_dims_[0], in_dims_[1], in_dims_[2], in_dims_[3],
                                                        pool_size_, stride_, Device::stream()),
                          "MaxPool2D::backward_relu");
            return dx;
        }

        void MaxPool2D::set_fused_forward(const std::vector<int64_t>& in_dims, const DeviceTensor& out,
                                          const DeviceTensor& idx)
        {
            in_dims_ = in_dims;
            fused_out_ = out;
            idx_ = idx;
        }

        DeviceTensor MaxPool2D::backward_relu_pooled(const DeviceTensor& g)
        {
            if (!idx_.defined() || !fused_out_.defined())
                throw std::runtime_error("MaxPool2D::backward_relu_pooled without a fused forward");
            if (g.size() != idx_.size()) throw std::runtime_error("MaxPool2D::backward: grad shape mismatch");
            DeviceTensor dx = DeviceTensor::empty(in_dims_);
            Device::check(cnhip_maxpool2d_backward_relu_pooled(g.data(), idx_.idata(), fused_out_.data(), dx.data(),
                                                               in_dims_[0], in_dims_[1], in_dims_[2], in_dims_[3],
                                                               pool_size_, stride_, Device::stream()),
                          "MaxPool2D::backward_relu_pooled");
            return dx;
        }

        Tensor<float, 4> MaxPool2D::forward(const Tensor<float, 4>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 4>();
        }
        Tensor<float, 4> MaxPool2D::backward(const Tensor<float, 4>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 4>();
        }
        const Tensor<int, 4> MaxPool2D::get_max_indices() const { return idx_.to_host<int, 4>(); }

        // ---------------------------------------------------------------- Flatten
        DeviceTensor Flatten::forward(const DeviceTensor& x)
        {
            if (x.rank() != 4) throw std::runtime_error("Flatten::forward: expected a 4-D input");
            for (int i = 0; i < 4; ++i) input_shape_[static_cast<size_t>(i)] = x.dimension(i);
            return x.reshape({x.dimension(0), x.dimension(1) * x.dimension(2) * x.dimension(3)});
        }
        DeviceTensor Flatten::backward(const DeviceTensor& g)
        {
            return g.reshape({input_shape_[0], input_shape_[1], input_shape_[2], input_shape_[3]});
        }
        Tensor<float, 2> Flatten::forward(const Tensor<float, 4>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 2>();
        }
        Tensor<float, 4> Flatten::backward(const Tensor<float, 2>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 4>();
        }
    } // namespace Layers
} // namespace CppNet
