// SequentialModel over device tensors (ref: src/CppNet/models/models.cpp:13-101).
#include "CppNet/models/models.hpp"

#include "CppNet/activations/relu.hpp"

#include <iostream>
#include <string>

namespace CppNet
{
    namespace Models
    {
        void SequentialModel::add_activation(std::shared_ptr<Activations::Activation> activation)
        {
            if (!activation) throw std::invalid_argument("Cannot add null activation to model");
            steps_.push_back(std::make_shared<detail::ActivationStep>(std::move(activation)));
        }

        DeviceTensor SequentialModel::forward(const DeviceTensor& input) { return forward_prefix(input, steps_.size()); }

        Activations::Activation* SequentialModel::last_activation() const
        {
            return steps_.empty() ? nullptr : steps_.back()->activation();
        }

        Layers::Linear* SequentialModel::step_linear(std::size_t i) const
        {
            return i < steps_.size() ? steps_[i]->linear() : nullptr;
        }

        Activations::Activation* SequentialModel::step_activation(std::size_t i) const
        {
            return i < steps_.size() ? steps_[i]->activation() : nullptr;
        }

        DeviceTensor SequentialModel::forward_prefix(const DeviceTensor& input, std::size_t count)
        {
            if (count > steps_.size()) throw std::out_of_range("SequentialModel::forward_prefix: too many steps");
            DeviceTensor x = input;
            for (std::size_t i = 0; i < count; ++i)
            {
                Activations::Activation* next = i + 1 < count ? steps_[i + 1]->activation() : nullptr;
                if (auto* relu = dynamic_cast<Activations::ReLU*>(next))
                {
                    if (Layers::Linear* lin = steps_[i]->linear())
                    {
                        x = lin->forward_act(x, CNHIP_ACT_RELU);
                        relu->set_output_cache(x);
                        ++i;
                        continue;
                    }
                    if (Layers::Conv2D* conv = steps_[i]->conv2d())
                    {
                        // Conv2D -> ReLU -> MaxPool2D: one call, the ReLU output not
                        // kept (the pool's backward masks with its own output)
                        Layers::MaxPool2D* mp = i + 2 < count ? steps_[i + 2]->maxpool() : nullptr;
                        if (mp)
                        {
                            x = conv->forward_relu_maxpool(x, *mp);
                            relu->set_output_cache(DeviceTensor());
                            i += 2;
                            continue;
                        }
                        x = conv->forward_relu(x);
                        relu->set_output_cache(x);
                        ++i;
                        continue;
                    }
                }
                x = steps_[i]->forward(x);
            }
            return x;
        }

        DeviceTensor SequentialModel::backward(const DeviceTensor& grad_output)
        {
            return backward_from(grad_output, 0, true, steps_.size());
        }

        void SequentialModel::backward_params(const DeviceTensor& grad_output)
        {
            backward_params_prefix(grad_output, steps_.size());
        }

        void SequentialModel::backward_params_prefix(const DeviceTensor& grad_output, std::size_t count)
        {
            if (count > steps_.size())
                throw std::out_of_range("SequentialModel::backward_params_prefix: too many steps");
            std::size_t first = 0;
            while (first < count && !steps_[first]->is_trainable()) ++first;
            if (first == count) return;  // nothing to train
            backward_from(grad_output, first, false, count);
        }

        // Runs steps end-1 .. first; step `first` computes its input gradient
        // only when input_grad is set.  Fusions with a ReLU at k-1 apply only
        // for k > first, where that ReLU's backward is part of the range.
        DeviceTensor SequentialModel::backward_from(const DeviceTensor& grad_output, std::size_t first,
                                                    bool input_grad, std::size_t end)
        {
            DeviceTensor g = grad_output;
            for (std::size_t k = end; k-- > first;)
            {
                if (k == first && !input_grad) return steps_[k]->backward_no_input_grad(g);
                // LSTM -> SequenceLast: the LSTM takes the last step's gradient
                // as it is, without the zeros of the other steps
                Layers::LSTM* lstm = k > first && steps_[k]->sequence_last() ? steps_[k - 1]->lstm() : nullptr;
                if (lstm)
                {
                    const bool dx = input_grad || k - 1 > first;
                    g = lstm->backward_last(g, dx);
                    if (!dx) return g;
                    --k;
                    continue;
                }
                // Conv2D -> ReLU -> MaxPool2D -> Flatten -> Linear: the backward
                // of the last four in one pass over the pooled output
                if (k >= first + 3 && (k - 3 > first || input_grad))
                {
                    Layers::Linear* lin = steps_[k]->linear();
                    Layers::MaxPool2D* mp = lin ? steps_[k - 2]->maxpool() : nullptr;
                    if (mp && steps_[k - 1]->flatten() &&
                        dynamic_cast<Activations::ReLU*>(steps_[k - 3]->activation()) &&
                        lin->fuses_maxpool_backward(g, *mp))
                    {
                        g = lin->backward_maxpool_relu(g, *mp);
                        k -= 3;
                        continue;
                    }
                }
                Activations::Activation* prev = k > first ? steps_[k - 1]->activation() : nullptr;
                auto* relu = dynamic_cast<Activations::ReLU*>(prev);
                Layers::MaxPool2D* fused_mp = steps_[k]->maxpool();
                // Conv2D -> ReLU -> MaxPool2D as the first trainable layers with
                // no input gradient wanted: the conv's parameter gradients
                // straight from the pooled gradient
                if (relu && fused_mp && fused_mp->fused_forward() && !input_grad && k == first + 2)
                {
                    Layers::Conv2D* conv = steps_[first]->conv2d();
                    if (conv && conv->fuses_pool_backward(g, *fused_mp))
                    {
                        conv->backward_params_maxpool_relu(g, *fused_mp);
                        return DeviceTensor();
                    }
                }
                if (relu && fused_mp && fused_mp->fused_forward())
                {
                    g = fused_mp->backward_relu_pooled(g);
                    --k;
                    continue;
                }
                if (relu && relu->output_cache().defined())
                {
                    if (Layers::Linear* lin = steps_[k]->linear())
                    {
                        g = lin->backward_act(g, CNHIP_ACT_RELU, relu->output_cache());
                        --k;
                        continue;
                    }
                    if (Layers::MaxPool2D* mp = steps_[k]->maxpool())
                    {
                        g = mp->backward_relu(g, relu->output_cache());
                        --k;
                        continue;
                    }
                }
                g = steps_[k]->backward(g);
            }
            return g;
        }

        Tensor<float, 2> SequentialModel::forward(const Tensor<float, 2>& input)
        {
            return forward(DeviceTensor::from_host(input)).to_host<float, 2>();
        }

        Tensor<float, 2> SequentialModel::backward(const Tensor<float, 2>& grad_output)
        {
            return backward(DeviceTensor::from_host(grad_output)).to_host<float, 2>();
        }

        std::shared_ptr<Layers::Layer> SequentialModel::get_layer(std::size_t index) const
        {
            if (index >= layers_.size())
                throw std::out_of_range("Layer index " + std::to_string(index) + " out of range (model has " +
                                        std::to_string(layers_.size()) + " layers)");
            return layers_[index];
        }

        void SequentialModel::update(Optimizers::Optimizer& optimizer, float learning_rate)
        {
            optimizer.begin_group();
            try
            {
                for (auto& s : steps_)
                    if (s->is_trainable()) s->step(optimizer, learning_rate);
            }
            catch (...)
            {
                optimizer.end_group();
                throw;
            }
            optimizer.end_group();
        }

        void SequentialModel::zero_grad()
        {
            for (auto& l : layers_) l->reset_grads();
        }

        void SequentialModel::summary() const
        {
            std::cout << "SequentialModel: " << steps_.size() << " steps, " << layers_.size()
                      << " parameterised layers (device gpu)\n";
        }
    } // namespace Models
} // namespace CppNet
