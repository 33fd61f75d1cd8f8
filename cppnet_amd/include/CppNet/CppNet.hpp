/**
 * @file CppNet.hpp
 * @brief Umbrella header of the MI355X gpu backend (ref: include/CppNet/CppNet.hpp).
 */
#ifndef CPPNET_HPP
#define CPPNET_HPP

#include "CppNet/core/device.hpp"
#include "CppNet/core/tensor.hpp"
#include "CppNet/utils/init.hpp"
#include "CppNet/utils/serialization.hpp"
#include "CppNet/utils/tensor_io.hpp"
#include "CppNet/utils/dataloader.hpp"
#include "CppNet/layers/layer.hpp"
#include "CppNet/layers/linear.hpp"
#include "CppNet/layers/conv2d.hpp"
#include "CppNet/layers/max_pool2d.hpp"
#include "CppNet/layers/flatten.hpp"
#include "CppNet/layers/lstm.hpp"
#include "CppNet/layers/gru.hpp"
#include "CppNet/layers/sequence_last.hpp"
#include "CppNet/layers/embedding.hpp"
#include "CppNet/layers/attention.hpp"
#include "CppNet/layers/batch_norm.hpp"
#include "CppNet/layers/mean_pool1d.hpp"
#include "CppNet/layers/residual.hpp"
#include "CppNet/layers/rnn.hpp"
#include "CppNet/layers/dropout.hpp"
#include "CppNet/layers/global_pool.hpp"
#include "CppNet/activations/activation.hpp"
#include "CppNet/activations/relu.hpp"
#include "CppNet/activations/sigmoid.hpp"
#include "CppNet/activations/tanh.hpp"
#include "CppNet/activations/gelu.hpp"
#include "CppNet/activations/leacky_relu.hpp"
#include "CppNet/activations/softmax.hpp"
#include "CppNet/losses/loss.hpp"
#include "CppNet/losses/binary_cross_entropy.hpp"
#include "CppNet/losses/mse.hpp"
#include "CppNet/losses/softmax_cross_entropy.hpp"
#include "CppNet/losses/categorical_cross_entropy.hpp"
#include "CppNet/losses/mae.hpp"
#include "CppNet/losses/huber.hpp"
#include "CppNet/optimizers/optimizer.hpp"
#include "CppNet/optimizers/adam.hpp"
#include "CppNet/optimizers/sgd.hpp"
#include "CppNet/optimizers/momentum.hpp"
#include "CppNet/optimizers/adagrad.hpp"
#include "CppNet/optimizers/mrs_prop.hpp"
#include "CppNet/models/models.hpp"

namespace CppNet
{
    /// The reference's has_cuda_support() (CppNet.hpp:127-134): true when a
    /// HIP device is visible to this process.
    inline bool has_cuda_support() { return Device::available(); }
    inline bool has_gpu_support() { return Device::available(); }
} // namespace CppNet
#endif
