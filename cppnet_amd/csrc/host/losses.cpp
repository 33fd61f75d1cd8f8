// Losses on device "gpu" (ref: src/CppNet/losses/binary_cross_entropy.cpp:
// 143-225, mse.cpp:102-161, softmax_cross_entropy.cpp:118-195).
#include <stdexcept>
#include <string>

#include "CppNet/layers/layer.hpp"
#include "CppNet/losses/binary_cross_entropy.hpp"
#include "CppNet/losses/mse.hpp"
#include "CppNet/losses/softmax_cross_entropy.hpp"

namespace CppNet
{
    namespace Losses
    {
        float DeviceScalar::get() const
        {
            if (!t_.defined()) throw std::runtime_error("DeviceScalar: no value");
            float v = 0.f;
            t_.copy_to_host(&v);
            return v;
        }

        float Loss::forward(const Tensor<float, 2>& p, const Tensor<float, 2>& t)
        {
            return forward(DeviceTensor::from_host(p), DeviceTensor::from_host(t)).get();
        }

        Tensor<float, 2> Loss::backward(const Tensor<float, 2>& p, const Tensor<float, 2>& t)
        {
            return backward(DeviceTensor::from_host(p), DeviceTensor::from_host(t)).to_host<float, 2>();
        }

        int reduction_code(const std::string& r, const char* who, bool allow_none)
        {
            if (r == "mean") return CNHIP_REDUCE_MEAN;
            if (r == "sum") return CNHIP_REDUCE_SUM;
            if (allow_none && r == "none") return -1;
            throw std::invalid_argument(std::string(who) + ": reduction must be \"mean\" or \"sum\"" +
                                        (allow_none ? " or \"none\"" : "") + ", got \"" + r + "\"");
        }

        static void require_same_shape(const DeviceTensor& p, const DeviceTensor& t, const char* who)
        {
            if (!p.defined() || !t.defined() || p.size() == 0)
                throw std::invalid_argument(std::string(who) + ": empty input");
            if (p.dims() != t.dims())
                throw std::invalid_argument(std::string(who) + ": predictions " + shape_str(p.dims()) +
                                            " and targets " + shape_str(t.dims()) + " differ");
        }

        // ---------------------------------------------------------------- BCE
        BinaryCrossEntropy::BinaryCrossEntropy(const std::string& reduction, bool from_logits,
                                               float pos_weight, const std::string& device)
            : reduction_(reduction), from_logits_(from_logits), pos_weight_(pos_weight), device_(device)
        {
            if (reduction_ != "mean" && reduction_ != "sum" && reduction_ != "none")
                throw std::runtime_error("Invalid reduction method: " + reduction_ +
                                         ". Must be 'mean', 'sum', or 'none'.");
            Layers::require_gpu_device(device_, "BinaryCrossEntropy");
        }

        // Host overloads keep the reference's target validation (targets in {0,1}).
        static void validate_bce(const Tensor<float, 2>& p, const Tensor<float, 2>& t)
        {
            if (p.dimension(0) != t.dimension(0) || p.dimension(1) != t.dimension(1))
                throw std::invalid_argument("Predictions and targets must have the same shape");
            for (int64_t i = 0; i < t.size(); ++i)
                if (t.data()[i] != 0.0f && t.data()[i] != 1.0f)
                    throw std::invalid_argument("Targets must be 0 or 1 for binary cross-entropy");
        }

        float BinaryCrossEntropy::forward(const Tensor<float, 2>& p, const Tensor<float, 2>& t)
        {
            validate_bce(p, t);
            return Loss::forward(p, t);
        }

        Tensor<float, 2> BinaryCrossEntropy::backward(const Tensor<float, 2>& p, const Tensor<float, 2>& t)
        {
            validate_bce(p, t);
            return Loss::backward(p, t);
        }

        DeviceScalar BinaryCrossEntropy::forward(const DeviceTensor& p, const DeviceTensor& t)
        {
            require_same_shape(p, t, "BinaryCrossEntropy::forward");
            // "none" returns the mean, as the reference's forward does.
            const int red = forward_reduction();
            DeviceTensor loss = DeviceTensor::empty({1});
            Device::check(cnhip_bce_forward(p.data(), t.data(), loss.data(), p.size(), red,
                                            Device::stream()),
                          "BinaryCrossEntropy::forward");
            return DeviceScalar(loss);
        }

        DeviceTensor BinaryCrossEntropy::backward(const DeviceTensor& p, const DeviceTensor& t)
        {
            require_same_shape(p, t, "BinaryCrossEntropy::backward");
            // only "mean" divides the gradient by the element count
            const int red = backward_reduction();
            DeviceTensor g = DeviceTensor::empty(p.dims());
            Device::check(cnhip_bce_backward(p.data(), t.data(), g.data(), p.size(), red,
                                             Device::stream()),
                          "BinaryCrossEntropy::backward");
            return g;
        }

        // ---------------------------------------------------------------- MSE
        MSE::MSE(const std::string& reduction, const std::string& device)
            : reduction_(reduction), device_(device)
        {
            reduction_code(reduction_, "MSE", true);
            Layers::require_gpu_device(device_, "MSE");
        }

        DeviceScalar MSE::forward(const DeviceTensor& p, const DeviceTensor& t)
        {
            require_same_shape(p, t, "MSE::forward");
            const int red = reduction_ == "mean" ? CNHIP_REDUCE_MEAN : CNHIP_REDUCE_SUM;
            DeviceTensor loss = DeviceTensor::empty({1});
            Device::check(cnhip_mse_forward(p.data(), t.data(), loss.data(), p.size(), red,
                                            Device::stream()),
                          "MSE::forward");
            return DeviceScalar(loss);
        }

        DeviceTensor MSE::backward(const DeviceTensor& p, const DeviceTensor& t)
        {
            require_same_shape(p, t, "MSE::backward");
            const int red = reduction_ == "mean" ? CNHIP_REDUCE_MEAN : CNHIP_REDUCE_SUM;
            DeviceTensor g = DeviceTensor::empty(p.dims());
            Device::check(cnhip_mse_backward(p.data(), t.data(), g.data(), p.size(), red,
                                             Device::stream()),
                          "MSE::backward");
            return g;
        }

        DeviceScalar MSE::forward_backward(const DeviceTensor& p, const DeviceTensor& t, DeviceTensor& grad)
        {
            require_same_shape(p, t, "MSE::forward_backward");
            if (static_cast<int64_t>(p.size()) > (int64_t{1} << 16))
            {
                DeviceScalar loss = forward(p, t);
                grad = backward(p, t);
                return loss;
            }
            const int red = reduction_ == "mean" ? CNHIP_REDUCE_MEAN : CNHIP_REDUCE_SUM;
            if (!grad.defined() || grad.dims() != p.dims()) grad = DeviceTensor::empty(p.dims());
            DeviceTensor loss = DeviceTensor::empty({1});
            Device::check(cnhip_mse_head(p.data(), t.data(), loss.data(), grad.data(), static_cast<int64_t>(p.size()),
                                         red, red, Device::stream()),
                          "MSE::forward_backward");
            return DeviceScalar(loss);
        }

        // ---------------------------------------------------------------- SoftmaxCE
        SoftmaxCrossEntropy::SoftmaxCrossEntropy(const std::string& reduction, const std::string& device)
            : reduction_(reduction), device_(device)
        {
            if (reduction_ != "mean" && reduction_ != "sum")
                throw std::invalid_argument("SoftmaxCrossEntropy: reduction must be \"mean\" or \"sum\"");
            Layers::require_gpu_device(device_, "SoftmaxCrossEntropy");
        }

        DeviceScalar SoftmaxCrossEntropy::forward_backward(const DeviceTensor& z, const DeviceTensor& t,
                                                           DeviceTensor& grad)
        {
            require_same_shape(z, t, "SoftmaxCrossEntropy::forward_backward");
            if (z.rank() != 2) throw std::invalid_argument("SoftmaxCrossEntropy: expected [batch, classes]");
            const int64_t B = z.dimension(0), C = z.dimension(1);
            if (!softmax_cache_.defined() || softmax_cache_.dims() != z.dims())
                softmax_cache_ = DeviceTensor::empty(z.dims());
            if (!grad.defined() || grad.dims() != z.dims()) grad = DeviceTensor::empty(z.dims());
            DeviceTensor loss = DeviceTensor::empty({1});
            Device::check(cnhip_softmax_ce_head(z.data(), t.data(), softmax_cache_.data(), loss.data(), grad.data(),
                                                B, C, reduction_code(reduction_, "SoftmaxCE", false),
                                                Device::stream()),
                          "SoftmaxCrossEntropy::forward_backward");
            return DeviceScalar(loss);
        }

        DeviceScalar SoftmaxCrossEntropy::forward(const DeviceTensor& z, const DeviceTensor& t)
        {
            require_same_shape(z, t, "SoftmaxCrossEntropy::forward");
            if (z.rank() != 2) throw std::invalid_argument("SoftmaxCrossEntropy: expected [batch, classes]");
            const int64_t B = z.dimension(0), C = z.dimension(1);
            if (!softmax_cache_.defined() || softmax_cache_.dims() != z.dims())
                softmax_cache_ = DeviceTensor::empty(z.dims());
            DeviceTensor loss = DeviceTensor::empty({1});
            Device::check(cnhip_softmax_ce_forward(z.data(), t.data(), softmax_cache_.data(), loss.data(),
                                                   B, C, reduction_code(reduction_, "SoftmaxCE", false),
                                                   Device::stream()),
                          "SoftmaxCrossEntropy::forward");
            return DeviceScalar(loss);
        }

        DeviceTensor SoftmaxCrossEntropy::backward(const DeviceTensor& z, const DeviceTensor& t)
        {
            require_same_shape(z, t, "SoftmaxCrossEntropy::backward");
            if (!softmax_cache_.defined() || softmax_cache_.dims() != z.dims()) forward(z, t);
            const int64_t B = z.dimension(0), C = z.dimension(1);
            DeviceTensor g = DeviceTensor::empty(z.dims());
            Device::check(cnhip_softmax_ce_backward(softmax_cache_.data(), t.data(), g.data(), B, C,
                                                    reduction_code(reduction_, "SoftmaxCE", false),
                                                    Device::stream()),
                          "SoftmaxCrossEntropy::backward");
            return g;
        }
    } // namespace Losses
} // namespace CppNet
