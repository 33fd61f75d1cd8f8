/**
 * @file batch_norm.hpp
 * @brief BatchNorm, device "gpu" (ref: include/CppNet/layers/batch_norm.hpp,
 *        src/CppNet/layers/batch_norm.cpp:25-401).
 *
 * x [N, F] ColMajor (a [B, S, D] activation is used through its free
 * [B*S, D] reshape).  Training mode (the default) normalises with the biased
 * batch variance and updates running stats (1 - momentum) r + momentum *
 * batch; eval() normalises with the running stats.  gamma = 1, beta = 0,
 * running mean 0, running var 1 at construction.  backward() OVERWRITES the
 * gradients (batch_norm.cpp:353-385, the batch statistics of the last
 * training forward); step() updates gamma then beta and clears the
 * gradients (batch_norm.cpp:390-401).
 */
#ifndef CPPNET_LAYERS_BATCH_NORM_HPP
#define CPPNET_LAYERS_BATCH_NORM_HPP

#include <string>

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Layers
    {
        class BatchNorm : public Layer
        {
        public:
            BatchNorm(int num_features, float momentum = 0.1f, float eps = 1e-5f,
                      const std::string& device = "gpu");

            Tensor<float, 2> forward(const Tensor<float, 2>& input);
            Tensor<float, 2> backward(const Tensor<float, 2>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);

            bool is_trainable() const override { return trainable_; }
            void step(Optimizers::Optimizer& optimizer, float learning_rate) override;
            void reset_grads() override { grads_zero_ = true; }
            void train() { training_ = true; }
            void eval() { training_ = false; }
            void freeze() { trainable_ = false; }
            void unfreeze() { trainable_ = true; }
            int get_num_features() const { return num_features_; }

            const Tensor<float, 1> get_gamma() const { return gamma_.to_host<float, 1>(); }
            const Tensor<float, 1> get_beta() const { return beta_.to_host<float, 1>(); }
            const Tensor<float, 1> get_grad_gamma() const;
            const Tensor<float, 1> get_grad_beta() const;
            const Tensor<float, 1> get_running_mean() const { return rmean_.to_host<float, 1>(); }
            const Tensor<float, 1> get_running_var() const { return rvar_.to_host<float, 1>(); }
            void set_gamma(const Tensor<float, 1>& g);
            void set_beta(const Tensor<float, 1>& b);
            void set_running_mean(const Tensor<float, 1>& m);
            void set_running_var(const Tensor<float, 1>& v);

            DeviceTensor& gamma() { return gamma_; }
            DeviceTensor& beta() { return beta_; }
            DeviceTensor& grad_gamma() { materialize_grads(); return ggamma_; }
            DeviceTensor& grad_beta() { materialize_grads(); return gbeta_; }

        private:
            void materialize_grads() const;
            int num_features_;
            float momentum_, eps_;
            bool training_ = true;
            bool trainable_ = true;
            std::string device_;
            DeviceTensor gamma_, beta_, ggamma_, gbeta_, rmean_, rvar_, bmean_, bvar_;
            DeviceTensor in_cache_, xhat_;
        };
    } // namespace Layers
} // namespace CppNet
#endif
