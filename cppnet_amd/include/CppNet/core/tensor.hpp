/**
 * @file tensor.hpp
 * @brief Host and device tensors of the gpu backend (ColMajor, fp32/int32).
 *
 * CppNet's API is written against Eigen::Tensor<float,R> (ColMajor).  Eigen
 * is not a dependency of this backend: CppNet::Tensor<T,R> below provides the
 * part of Eigen's Tensor interface the layer API and its callers use
 * (dimension, dimensions, size, data, operator(), setZero, setConstant,
 * setValues, resize) with the same ColMajor memory order, so host data moves
 * to and from the device without reordering.
 *
 * CppNet::DeviceTensor is a shape plus a reference-counted HBM buffer from
 * the caching allocator (device.hpp).  Layers take and return DeviceTensors
 * so activations, gradients and optimizer state stay resident in HBM.
 */
#ifndef CPPNET_CORE_TENSOR_HPP
#define CPPNET_CORE_TENSOR_HPP

#include <array>
#include <cstdint>
#include <initializer_list>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "CppNet/core/device.hpp"

namespace CppNet
{
    template <typename T, int R>
    class Tensor
    {
    public:
        using Index = int64_t;
        using Dimensions = std::array<Index, R>;

        Tensor() { dims_.fill(0); }

        template <typename... I,
                  typename = std::enable_if_t<sizeof...(I) == R && R != 0>>
        explicit Tensor(I... dims) : dims_{static_cast<Index>(dims)...}
        {
            data_.assign(static_cast<size_t>(count(dims_)), T(0));
        }

        explicit Tensor(const Dimensions& dims) : dims_(dims)
        {
            data_.assign(static_cast<size_t>(count(dims_)), T(0));
        }

        // Assignment only to lvalues.  The layers' state getters return host
        // copies (the state lives in HBM) as const values, so reference code
        // that writes through a getter it expects to return a reference
        // (`bn.get_gamma() = g`, `lin.get_weights()(0, 0) = w`) fails to
        // compile here instead of writing into a discarded temporary; such
        // code uses the setters (set_gamma, set_weights, ...).
        Tensor(const Tensor&) = default;
        Tensor(Tensor&&) noexcept = default;
        Tensor& operator=(const Tensor&) & = default;
        Tensor& operator=(Tensor&&) & noexcept = default;

        Index dimension(int i) const { return dims_.at(static_cast<size_t>(i)); }
        const Dimensions& dimensions() const { return dims_; }
        Index size() const { return static_cast<Index>(data_.size()); }
        static constexpr int NumDimensions = R;

        T* data() { return data_.data(); }
        const T* data() const { return data_.data(); }

        template <typename... I>
        T& operator()(I... idx) { return data_[static_cast<size_t>(offset(idx...))]; }
        template <typename... I>
        const T& operator()(I... idx) const { return data_[static_cast<size_t>(offset(idx...))]; }

        Tensor& setZero() { return setConstant(T(0)); }
        Tensor& setConstant(T v)
        {
            for (auto& x : data_) x = v;
            return *this;
        }

        template <typename... I>
        void resize(I... dims)
        {
            static_assert(sizeof...(I) == R, "resize: rank mismatch");
            dims_ = Dimensions{static_cast<Index>(dims)...};
            data_.assign(static_cast<size_t>(count(dims_)), T(0));
        }

        /// setValues with logical (row-by-row) nesting, as Eigen's.
        template <int RR = R, typename = std::enable_if_t<RR == 1>>
        Tensor& setValues(std::initializer_list<T> v)
        {
            if (static_cast<Index>(v.size()) != dims_[0])
                throw std::invalid_argument("Tensor::setValues: size mismatch");
            Index i = 0;
            for (T x : v) data_[static_cast<size_t>(i++)] = x;
            return *this;
        }
        template <int RR = R, typename = std::enable_if_t<RR == 2>>
        Tensor& setValues(std::initializer_list<std::initializer_list<T>> v)
        {
            if (static_cast<Index>(v.size()) != dims_[0])
                throw std::invalid_argument("Tensor::setValues: row count mismatch");
            Index r = 0;
            for (const auto& row : v)
            {
                if (static_cast<Index>(row.size()) != dims_[1])
                    throw std::invalid_argument("Tensor::setValues: column count mismatch");
                Index c = 0;
                for (T x : row) (*this)(r, c++) = x;
                ++r;
            }
            return *this;
        }

    private:
        static Index count(const Dimensions& d)
        {
            Index n = 1;
            for (Index x : d)
            {
                if (x < 0) throw std::invalid_argument("Tensor: negative dimension");
                n *= x;
            }
            return n;
        }
        template <typename... I>
        Index offset(I... idx) const
        {
            static_assert(sizeof...(I) == R, "Tensor: wrong number of indices");
            const Index ix[R] = {static_cast<Index>(idx)...};
            Index off = 0;
            for (int d = R - 1; d >= 0; --d) off = off * dims_[d] + ix[d];  // ColMajor
            return off;
        }

        Dimensions dims_;
        std::vector<T> data_;
    };

    /**
     * A ColMajor device tensor: dims + a shared HBM buffer.  Copies share the
     * buffer (views); reshape() is free, as in ColMajor Eigen.
     */
    class DeviceTensor
    {
    public:
        DeviceTensor() = default;

        static DeviceTensor empty(std::vector<int64_t> dims, int elem_bytes = 4);
        static DeviceTensor zeros(std::vector<int64_t> dims, int elem_bytes = 4);

        template <typename T, int R>
        static DeviceTensor from_host(const Tensor<T, R>& h)
        {
            static_assert(sizeof(T) == 4, "DeviceTensor holds 4-byte elements");
            std::vector<int64_t> dims(h.dimensions().begin(), h.dimensions().end());
            DeviceTensor t = empty(dims);
            t.copy_from_host(h.data());
            return t;
        }

        template <typename T, int R>
        Tensor<T, R> to_host() const
        {
            static_assert(sizeof(T) == 4, "DeviceTensor holds 4-byte elements");
            if (rank() != R) throw std::invalid_argument("DeviceTensor::to_host: rank mismatch");
            typename Tensor<T, R>::Dimensions d;
            for (int i = 0; i < R; ++i) d[static_cast<size_t>(i)] = dims_[static_cast<size_t>(i)];
            Tensor<T, R> h(d);
            copy_to_host(h.data());
            return h;
        }

        void copy_from_host(const void* src);           ///< synchronous H2D of size() elements
        void copy_to_host(void* dst) const;              ///< synchronises the stream, D2H
        void copy_from_device(const DeviceTensor& src);  ///< async D2D, same size required
        void fill_zero();                                ///< async

        float* data() { return reinterpret_cast<float*>(ptr_); }
        const float* data() const { return reinterpret_cast<const float*>(ptr_); }
        int32_t* idata() { return reinterpret_cast<int32_t*>(ptr_); }
        const int32_t* idata() const { return reinterpret_cast<const int32_t*>(ptr_); }

        int rank() const { return static_cast<int>(dims_.size()); }
        int64_t dimension(int i) const { return dims_.at(static_cast<size_t>(i)); }
        const std::vector<int64_t>& dims() const { return dims_; }
        int64_t size() const;
        bool defined() const { return static_cast<bool>(buf_); }

        /// Same buffer, new ColMajor shape (element count must match).
        DeviceTensor reshape(std::vector<int64_t> dims) const;
        /// Same buffer, elements [offset, offset + prod(dims)) as a tensor of
        /// shape dims (the packed-parameter views of MultiHeadAttention).
        DeviceTensor view(int64_t offset, std::vector<int64_t> dims) const;

    private:
        std::vector<int64_t> dims_;
        std::shared_ptr<Device::Buffer> buf_;
        void* ptr_ = nullptr;
    };

    std::string shape_str(const std::vector<int64_t>& dims);
} // namespace CppNet

#endif
