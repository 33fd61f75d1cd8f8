/**
 * @file residual.hpp
 * @brief Residual, device "gpu" (ref: include/CppNet/layers/residual.hpp,
 *        src/CppNet/layers/residual.cpp:23-159).
 *
 * out = block(x) + shortcut(x) on [batch, features].  As in the reference,
 * only the Linear layers of the block are applied (other layer types are
 * skipped), and the shortcut is x itself or, when in_features !=
 * out_features, a bias-free trainable Linear projection.  backward() sums
 * the two paths' gradients; step() steps the trainable block layers and the
 * projection; reset_grads() resets the Linear layers.
 */
#ifndef CPPNET_LAYERS_RESIDUAL_HPP
#define CPPNET_LAYERS_RESIDUAL_HPP

#include <memory>
#include <string>
#include <vector>

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"
#include "CppNet/layers/linear.hpp"

namespace CppNet
{
    namespace Layers
    {
        class Residual : public Layer
        {
        public:
            Residual(std::vector<std::shared_ptr<Layer>> block, int in_features, int out_features,
                     const std::string& device = "gpu");
            Tensor<float, 2> forward(const Tensor<float, 2>& input);
            Tensor<float, 2> backward(const Tensor<float, 2>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);
            bool is_trainable() const override { return true; }
            void step(Optimizers::Optimizer& optimizer, float learning_rate) override;
            void reset_grads() override;
            std::size_t num_block_layers() const { return block_.size(); }
            Layer* block_layer(std::size_t i) const { return block_.at(i).get(); }
            bool has_projection() const { return projection_ != nullptr; }
            Linear* projection() { return projection_.get(); }

        private:
            std::vector<std::shared_ptr<Layer>> block_;
            std::shared_ptr<Linear> projection_;
            int in_features_, out_features_;
            std::string device_;
        };
    } // namespace Layers
} // namespace CppNet
#endif
