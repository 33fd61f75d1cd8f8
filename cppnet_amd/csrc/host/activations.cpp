// ReLU / Sigmoid / Tanh on device "gpu" (ref: src/CppNet/activations/
// relu.cpp:97-225, sigmoid.cpp:97-231, tanh.cpp:100-219).  Each caches its
// OUTPUT in forward and derives the backward mask/slope from it.
#include <stdexcept>
#include <string>

#include "CppNet/activations/relu.hpp"
#include "CppNet/activations/sigmoid.hpp"
#include "CppNet/activations/tanh.hpp"
#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Activations
    {
        Tensor<float, 2> Activation::forward(const Tensor<float, 2>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 2>();
        }
        Tensor<float, 2> Activation::backward(const Tensor<float, 2>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 2>();
        }
        Tensor<float, 4> Activation::forward(const Tensor<float, 4>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 4>();
        }
        Tensor<float, 4> Activation::backward(const Tensor<float, 4>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 4>();
        }

        DeviceTensor OutputCachedActivation::forward(const DeviceTensor& x)
        {
            if (!x.defined() || x.size() == 0)
                throw std::runtime_error(std::string(name_) + ": empty input");
            DeviceTensor y = DeviceTensor::empty(x.dims());
            Device::check(launch_forward(x.data(), y.data(), x.size()), name_);
            out_cache_ = y;
            return y;
        }

        DeviceTensor OutputCachedActivation::backward(const DeviceTensor& g)
        {
            if (!g.defined() || g.size() == 0)
                throw std::runtime_error(std::string(name_) + ": empty grad");
            if (!out_cache_.defined() || out_cache_.size() != g.size())
                throw std::runtime_error(std::string(name_) + ": backward before forward or shape mismatch");
            DeviceTensor dx = DeviceTensor::empty(g.dims());
            Device::check(launch_backward(out_cache_.data(), g.data(), dx.data(), g.size()), name_);
            return dx;
        }

        ReLU::ReLU(const std::string& device) : OutputCachedActivation("ReLU")
        {
            Layers::require_gpu_device(device, "ReLU");
        }
        int ReLU::launch_forward(const float* x, float* y, int64_t n)
        {
            return cnhip_relu_forward(x, y, n, Device::stream());
        }
        int ReLU::launch_backward(const float* y, const float* dy, float* dx, int64_t n)
        {
            return cnhip_relu_backward(y, dy, dx, n, Device::stream());
        }

        Sigmoid::Sigmoid(const std::string& device) : OutputCachedActivation("Sigmoid")
        {
            Layers::require_gpu_device(device, "Sigmoid");
        }
        int Sigmoid::launch_forward(const float* x, float* y, int64_t n)
        {
            return cnhip_sigmoid_forward(x, y, n, Device::stream());
        }
        int Sigmoid::launch_backward(const float* y, const float* dy, float* dx, int64_t n)
        {
            return cnhip_sigmoid_backward(y, dy, dx, n, Device::stream());
        }

        Tanh::Tanh(const std::string& device) : OutputCachedActivation("Tanh")
        {
            Layers::require_gpu_device(device, "Tanh");
        }
        int Tanh::launch_forward(const float* x, float* y, int64_t n)
        {
            return cnhip_tanh_forward(x, y, n, Device::stream());
        }
        int Tanh::launch_backward(const float* y, const float* dy, float* dx, int64_t n)
        {
            return cnhip_tanh_backward(y, dy, dx, n, Device::stream());
        }
    } // namespace Activations
} // namespace CppNet
