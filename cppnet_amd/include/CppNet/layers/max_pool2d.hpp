/**
 * @file max_pool2d.hpp
 * @brief MaxPool2D, device "gpu" (ref: include/CppNet/layers/max_pool2d.hpp:29-52,
 *        src/CppNet/layers/max_pool2d.cpp:25-131).
 *
 * stride <= 0 means stride = pool_size; HO = (H - pool)/stride + 1, no
 * padding.  forward() keeps the int32 window-local argmax ph*pool + pw of the
 * first maximum (strict >) in HBM; backward() routes dY through it.
 */
#ifndef CPPNET_LAYERS_MAX_POOL2D_HPP
#define CPPNET_LAYERS_MAX_POOL2D_HPP

#include <string>

#include "CppNet/core/tensor.hpp"
#include "CppNet/layers/layer.hpp"

namespace CppNet
{
    namespace Layers
    {
        class MaxPool2D : public Layer
        {
        public:
            MaxPool2D(int pool_size = 2, int stride = -1, const std::string& device = "gpu");
            Tensor<float, 4> forward(const Tensor<float, 4>& input);
            Tensor<float, 4> backward(const Tensor<float, 4>& grad_output);
            DeviceTensor forward(const DeviceTensor& input);
            DeviceTensor backward(const DeviceTensor& grad_output);
            /// backward() followed by the backward of the ReLU whose output y
            /// is this layer's input: dX * [y > 0] in one pass, equal to the
            /// two calls.
            DeviceTensor backward_relu(const DeviceTensor& grad_output, const DeviceTensor& relu_out);
            /// Records a forward that Conv2D::forward_relu_maxpool ran for this
            /// layer: its input dims (the conv output's), pooled output and argmax.
            void set_fused_forward(const std::vector<int64_t>& in_dims, const DeviceTensor& out,
                                   const DeviceTensor& idx);
            /// Whether the last forward was fused (no ReLU output was kept).
            bool fused_forward() const { return fused_out_.defined(); }
            /// Pooled output of the last fused forward (undefined otherwise).
            const DeviceTensor& pooled_output() const { return fused_out_; }
            /// Input dims [N, C, H, W] of the last fused forward.
            const std::vector<int64_t>& input_dims() const { return in_dims_; }
            /// backward_relu() for a fused forward: the ReLU mask from this
            /// layer's own output.
            DeviceTensor backward_relu_pooled(const DeviceTensor& grad_output);
            bool is_trainable() const override { return false; }
            void step(Optimizers::Optimizer&, float) override {}
            int get_pool_size() const { return pool_size_; }
            int get_stride() const { return stride_; }
            /// int32 argmax of the last forward, [N, C, HO, WO]
            const DeviceTensor& max_indices() const { return idx_; }
            const Tensor<int, 4> get_max_indices() const;

        private:
            int pool_size_, stride_;
            std::string device_;
            DeviceTensor idx_;
            DeviceTensor fused_out_;  // pooled output of a fused forward, else undefined
            std::vector<int64_t> in_dims_;
        };
    } // namespace Layers
} // namespace CppNet
#endif
