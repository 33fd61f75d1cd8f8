/**
 * @file tensor_io.hpp
 * @brief NumPy .npy v1.0 files of float32 tensors
 *        (ref: include/CppNet/utils/tensor_io.hpp, src/CppNet/utils/tensor_io.cpp:29-170).
 *
 * The header is the reference's: magic, version 1.0, a little-endian uint16
 * length and the dict `{'descr': '<f4', 'fortran_order': ..., 'shape': (...), }`
 * space-padded so that the data starts at a multiple of 64 bytes.
 *
 * One deliberate difference: the data written is the tensor's ColMajor
 * memory, so the writer says `'fortran_order': True`; numpy.load then returns
 * the logical tensor.  (The reference writes the same bytes under `False`,
 * tensor_io.cpp:33, which numpy reads as a reshuffled array.)  The readers
 * follow the file's flag: Fortran-order data is taken as is, C-order data is
 * reordered into ColMajor.  raw_colmajor = true takes the data as ColMajor
 * whatever the flag says -- what the reference's reader does, for files the
 * reference wrote.
 */
#ifndef CPPNET_UTILS_TENSOR_IO_HPP
#define CPPNET_UTILS_TENSOR_IO_HPP

#include <cstdint>
#include <string>
#include <vector>

#include "CppNet/core/tensor.hpp"

namespace CppNet
{
    namespace Utils
    {
        void save_npy(const std::string& path, const Tensor<float, 1>& tensor);
        void save_npy(const std::string& path, const Tensor<float, 2>& tensor);
        void save_npy(const std::string& path, const Tensor<float, 3>& tensor);
        void save_npy(const std::string& path, const Tensor<float, 4>& tensor);
        /// A device tensor (one device-to-host copy).
        void save_npy(const std::string& path, const DeviceTensor& tensor);

        Tensor<float, 1> load_npy_1d(const std::string& path, bool raw_colmajor = false);
        Tensor<float, 2> load_npy_2d(const std::string& path, bool raw_colmajor = false);
        Tensor<float, 3> load_npy_3d(const std::string& path, bool raw_colmajor = false);
        Tensor<float, 4> load_npy_4d(const std::string& path, bool raw_colmajor = false);

        /// Untyped forms: ColMajor data of `dims` (any rank >= 1).
        void save_npy_raw(const std::string& path, const float* colmajor, const std::vector<int64_t>& dims);
        std::vector<float> load_npy_raw(const std::string& path, std::vector<int64_t>& dims,
                                        bool raw_colmajor = false);
    } // namespace Utils
} // namespace CppNet

#endif
