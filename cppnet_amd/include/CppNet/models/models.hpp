/**
 * @file models.hpp
 * @brief SequentialModel (ref: include/CppNet/models/models.hpp:116-218,
 *        src/CppNet/models/models.cpp:13-101) over device tensors.
 *
 * Steps run in insertion order; backward in reverse.  A Linear or Conv2D
 * followed by ReLU runs as one GEMM with the ReLU in its epilogue, and the
 * next Linear's input-gradient GEMM -- or the backward of a MaxPool2D that
 * follows the ReLU -- applies the ReLU mask (same arithmetic as the separate
 * calls).  Conv2D -> ReLU -> MaxPool2D runs as one forward call, and a
 * Linear head on its flattened output takes the backward of the Linear,
 * Flatten, pool and ReLU in one pass.
 * GELU is not fused: its erfc epilogue measured slower than a separate pass
 * on MI355X.  backward() returns the gradient of the model input, as the
 * reference does; backward_params() is the training step's variant: it
 * stops at the first trainable layer and skips that layer's input-gradient
 * product (the input is data, nothing consumes its gradient), leaving every
 * parameter gradient identical.  zero_grad() resets
 * every layer's gradients; update() steps every trainable layer, with all of
 * the optimizer's updates fused into one launch (begin_group/end_group).
 */
#ifndef CPPNET_MODELS_MODELS_HPP
#define CPPNET_MODELS_MODELS_HPP

#include <memory>
#include <stdexcept>
#include <type_traits>
#include <vector>

#include "CppNet/activations/activation.hpp"
#include "CppNet/layers/conv2d.hpp"
#include "CppNet/layers/flatten.hpp"
#include "CppNet/layers/linear.hpp"
#include "CppNet/layers/lstm.hpp"
#include "CppNet/layers/max_pool2d.hpp"
#include "CppNet/layers/sequence_last.hpp"
#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"
#include "CppNet/optimizers/optimizer.hpp"

namespace CppNet
{
    namespace detail
    {
        class Step
        {
        public:
            virtual DeviceTensor forward(const DeviceTensor& input) = 0;
            virtual DeviceTensor backward(const DeviceTensor& grad_output) = 0;
            virtual bool is_trainable() const = 0;
            virtual void step(Optimizers::Optimizer& optimizer, float learning_rate) = 0;
            /// Parameter gradients only; returns an undefined tensor where
            /// the layer can skip its input gradient.
            virtual DeviceTensor backward_no_input_grad(const DeviceTensor& g) { return backward(g); }
            virtual Layers::Linear* linear() { return nullptr; }
            virtual Layers::MaxPool2D* maxpool() { return nullptr; }
            virtual Layers::Flatten* flatten() { return nullptr; }
            virtual Layers::Conv2D* conv2d() { return nullptr; }
            virtual Layers::LSTM* lstm() { return nullptr; }
            virtual Layers::SequenceLast* sequence_last() { return nullptr; }
            virtual Activations::Activation* activation() { return nullptr; }
            virtual ~Step() = default;
        };

        template <typename L, typename = void>
        struct has_optional_input_grad : std::false_type
        {
        };
        template <typename L>
        struct has_optional_input_grad<
            L, std::void_t<decltype(std::declval<L&>().backward(std::declval<const DeviceTensor&>(), false))>>
            : std::true_type
        {
        };

        template <typename LayerT>
        class LayerStep : public Step
        {
        public:
            explicit LayerStep(std::shared_ptr<LayerT> layer) : layer_(std::move(layer)) {}
            DeviceTensor forward(const DeviceTensor& x) override { return layer_->forward(x); }
            DeviceTensor backward(const DeviceTensor& g) override { return layer_->backward(g); }
            DeviceTensor backward_no_input_grad(const DeviceTensor& g) override
            {
                if constexpr (has_optional_input_grad<LayerT>::value)
                    return layer_->backward(g, false);
                else
                    return layer_->backward(g);
            }
            bool is_trainable() const override { return layer_->is_trainable(); }
            void step(Optimizers::Optimizer& o, float lr) override { layer_->step(o, lr); }
            Layers::Linear* linear() override { return dynamic_cast<Layers::Linear*>(layer_.get()); }
            Layers::MaxPool2D* maxpool() override { return dynamic_cast<Layers::MaxPool2D*>(layer_.get()); }
            Layers::Flatten* flatten() override { return dynamic_cast<Layers::Flatten*>(layer_.get()); }
            Layers::Conv2D* conv2d() override { return dynamic_cast<Layers::Conv2D*>(layer_.get()); }
            Layers::LSTM* lstm() override { return dynamic_cast<Layers::LSTM*>(layer_.get()); }
            Layers::SequenceLast* sequence_last() override
            {
                return dynamic_cast<Layers::SequenceLast*>(layer_.get());
            }

        private:
            std::shared_ptr<LayerT> layer_;
        };

        class ActivationStep : public Step
        {
        public:
            explicit ActivationStep(std::shared_ptr<Activations::Activation> a) : act_(std::move(a)) {}
            DeviceTensor forward(const DeviceTensor& x) override { return act_->forward(x); }
            DeviceTensor backward(const DeviceTensor& g) override { return act_->backward(g); }
            bool is_trainable() const override { return false; }
            void step(Optimizers::Optimizer&, float) override {}
            Activations::Activation* activation() override { return act_.get(); }

        private:
            std::shared_ptr<Activations::Activation> act_;
        };
    } // namespace detail

    namespace Models
    {
        class SequentialModel
        {
        public:
            SequentialModel() = default;

            template <typename LayerT,
                      typename = std::enable_if_t<std::is_same<
                          std::decay_t<decltype(std::declval<LayerT>().forward(
                              std::declval<const DeviceTensor&>()))>,
                          DeviceTensor>::value>>
            void add_layer(std::shared_ptr<LayerT> layer)
            {
                if (!layer) throw std::invalid_argument("Cannot add null layer to model");
                steps_.push_back(std::make_shared<detail::LayerStep<LayerT>>(layer));
                layers_.push_back(layer);
            }
            void add_activation(std::shared_ptr<Activations::Activation> activation);

            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);
            void backward_params(const DeviceTensor& grad_output);
            /// forward through steps [0, count) only
            DeviceTensor forward_prefix(const DeviceTensor& input, std::size_t count);
            /// backward_params over steps [0, count): grad_output is the
            /// gradient of step count-1's output
            void backward_params_prefix(const DeviceTensor& grad_output, std::size_t count);
            /// the activation of the last step, or null
            Activations::Activation* last_activation() const;
            /// step i's Linear layer / activation, or null (i < num_steps())
            Layers::Linear* step_linear(std::size_t i) const;
            Activations::Activation* step_activation(std::size_t i) const;
            Tensor<float, 2> forward(const Tensor<float, 2>& input);
            Tensor<float, 2> backward(const Tensor<float, 2>& grad_output);

            std::size_t num_layers() const { return layers_.size(); }
            std::size_t num_steps() const { return steps_.size(); }
            std::shared_ptr<Layers::Layer> get_layer(std::size_t index) const;
            void update(Optimizers::Optimizer& optimizer, float learning_rate);
            void zero_grad();
            void summary() const;

        private:
            DeviceTensor backward_from(const DeviceTensor& grad_output, std::size_t first, bool input_grad,
                                       std::size_t end);
            std::vector<std::shared_ptr<detail::Step>> steps_;
            std::vector<std::shared_ptr<Layers::Layer>> layers_;
        };
    } // namespace Models
} // namespace CppNet
#endif
