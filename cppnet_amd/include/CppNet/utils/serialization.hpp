/**
 * @file serialization.hpp
 * @brief Model files (ref: include/CppNet/utils/serialization.hpp,
 *        src/CppNet/utils/serialization.cpp:26-256).
 *
 * Tensor record: int32 ndims, int32 dims[ndims], float32 data (ColMajor,
 * Eigen's order), little-endian.  save_tensor / load_tensor_* hold one record.
 *
 * save_model / load_model: the reference's "CNET" file, byte for byte:
 *   int32 magic 0x434E4554, int32 layer count, then per TRAINABLE layer an
 *   int32 type id and its tensors -- Linear 1: weights [in, out], biases
 *   [out] if it has them; BatchNorm 2: gamma, beta, running mean, running
 *   var; Embedding 3: the [vocab, dim] table; any other trainable layer 0
 *   and nothing else.  load_model fills the model's trainable layers in order
 *   and ignores what follows the records.
 *
 * save_checkpoint / load_checkpoint (no counterpart in the reference): the
 * CNET file above followed by an extension the reference's load_model never
 * reads, so that a checkpoint still loads there.  Extension:
 *   int32 magic 0x434E5831 ("CNX1"), int32 parameter count P, then per
 *   parameter of every trainable layer (step() order) a tensor record of its
 *   device-resident values; int32 optimizer kind (-1 none, 0 Adam, 1 SGD,
 *   2 Momentum, 3 Adagrad, 4 RMSProp), int32 state tensors per parameter S,
 *   then per parameter int32 present, int32 step count and S tensor records.
 * With it a run resumes exactly: the Conv2D / recurrent / attention weights
 * the CNET records skip and the optimizer's per-parameter state and step
 * counts are restored too.
 */
#ifndef CPPNET_UTILS_SERIALIZATION_HPP
#define CPPNET_UTILS_SERIALIZATION_HPP

#include <string>
#include <vector>

#include "CppNet/core/tensor.hpp"

namespace CppNet
{
    namespace Models
    {
        class SequentialModel;
    }
    namespace Layers
    {
        class Layer;
    }
    namespace Optimizers
    {
        class Optimizer;
    }

    namespace Utils
    {
        void save_tensor(const std::string& path, const Tensor<float, 2>& tensor);
        Tensor<float, 2> load_tensor_2d(const std::string& path);
        void save_tensor(const std::string& path, const Tensor<float, 1>& tensor);
        Tensor<float, 1> load_tensor_1d(const std::string& path);

        void save_model(const std::string& path, const Models::SequentialModel& model);
        void load_model(const std::string& path, Models::SequentialModel& model);

        void save_checkpoint(const std::string& path, const Models::SequentialModel& model,
                             const Optimizers::Optimizer* optimizer);
        void load_checkpoint(const std::string& path, Models::SequentialModel& model,
                             Optimizers::Optimizer* optimizer);

        /// The same files over an explicit layer sequence (a harness that
        /// composes layers without a SequentialModel).
        void save_layers(const std::string& path, const std::vector<Layers::Layer*>& layers,
                         const Optimizers::Optimizer* optimizer, bool extension);
        void load_layers(const std::string& path, const std::vector<Layers::Layer*>& layers,
                         Optimizers::Optimizer* optimizer, bool extension);
    } // namespace Utils
} // namespace CppNet

#endif
