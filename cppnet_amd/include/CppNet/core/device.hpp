/**
 * @file device.hpp
 * @brief Device runtime of the gpu backend: status checking, the stream all
 *        layers enqueue on, and a caching HBM allocator.
 *
 * The reference allocates and frees device memory inside every "gpu" layer
 * call (e.g. relu.cpp:229-246, conv2d.cpp:224-259).  Here every device buffer
 * comes from one caching allocator: a freed block returns to a size-keyed
 * cache and is handed out again to the next request of a similar size, so a
 * training loop reaches a steady state with no hipMalloc/hipFree at all.
 * Blocks are recycled in stream order, which is safe because all work of the
 * backend is enqueued on the single stream returned by Device::stream().
 */
#ifndef CPPNET_CORE_DEVICE_HPP
#define CPPNET_CORE_DEVICE_HPP

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>

#include "cnhip.h"

namespace CppNet
{
    namespace Device
    {
        /// Thrown for any non-zero cnhip status; what() carries cnhip_last_error().
        class Error : public std::runtime_error
        {
        public:
            Error(int status, const std::string& msg)
                : std::runtime_error(msg), status_(status) {}
            int status() const { return status_; }

        private:
            int status_;
        };

        /// Throws Error when status != CNHIP_OK.
        void check(int status, const char* context = nullptr);

        /// The stream every backend kernel is enqueued on (NULL = default stream).
        cnhip_stream_t stream();
        void set_stream(cnhip_stream_t s);
        void synchronize();

        /// True when a HIP device is visible (cf. CppNet.hpp has_cuda_support()).
        bool available();

        /// A block of device memory owned by the caching allocator.
        class Buffer
        {
        public:
            explicit Buffer(size_t bytes);
            ~Buffer();
            Buffer(const Buffer&) = delete;
            Buffer& operator=(const Buffer&) = delete;
            void* get() const { return ptr_; }
            size_t bytes() const { return bytes_; }

        private:
            void* ptr_ = nullptr;
            size_t bytes_ = 0;   // requested
            size_t block_ = 0;   // cached block size
            uint64_t pool_ = 0;  // graph pool it belongs to (0: the general cache)
        };

        std::shared_ptr<Buffer> allocate(size_t bytes);

        struct AllocatorStats
        {
            size_t device_bytes;   ///< bytes obtained from hipMalloc
            size_t cached_bytes;   ///< bytes idle in the cache
            size_t hip_mallocs;    ///< number of hipMalloc calls so far
        };
        AllocatorStats allocator_stats();
        /// Returns idle cached blocks to HIP (synchronises the device first).
        void empty_cache();

        /**
         * Graph pools: memory a captured graph refers to.  While a pool is
         * open (a capture of Device::stream() is running), every block handed
         * out belongs to the pool, and every block released goes to the
         * pool's own idle list (the captured kernels may refer to it).  Blocks
         * of a live pool are never handed to allocations made outside its
         * capture, so work enqueued between replays cannot be given memory
         * that a replay writes.  release_pool() (after the graph is destroyed)
         * moves the pool's idle blocks to the general cache; its blocks still
         * in use go there when released.
         */
        uint64_t open_pool();
        void close_pool();
        void release_pool(uint64_t id);
    } // namespace Device
} // namespace CppNet

#endif
