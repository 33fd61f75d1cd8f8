// Device runtime of the C++ host layer: status -> exception mapping, the
// backend stream, and the caching HBM allocator (see core/device.hpp).
#include "CppNet/core/device.hpp"

#include <map>
#include <mutex>
#include <string>

#include "CppNet/core/tensor.hpp"

namespace CppNet
{
    namespace Device
    {
        void check(int status, const char* context)
        {
            if (status == CNHIP_OK) return;
            std::string msg = cnhip_last_error();
            if (context) msg = std::string(context) + ": " + msg;
            throw Error(status, msg);
        }

        namespace
        {
            cnhip_stream_t g_stream = nullptr;

            // Size-keyed cache of idle blocks.  Leaked on purpose: buffers held
            // by static objects may be released after any static destructor.
            // Idle blocks are keyed by the stream they were released on: a
            // block may still be read by in-flight work of that stream, so it
            // is only handed out again to work enqueued on the same stream.
            struct Pool
            {
                cnhip_stream_t stream = nullptr;  // the captured stream
                std::multimap<size_t, void*> idle;
            };
            struct Cache
            {
                std::mutex mu;
                std::map<cnhip_stream_t, std::multimap<size_t, void*>> idle;
                std::map<uint64_t, Pool> pools;  // live graph pools
                uint64_t open = 0;               // pool of the running capture, 0 if none
                uint64_t next_pool = 1;
                size_t device_bytes = 0;
                size_t cached_bytes = 0;
                size_t mallocs = 0;
            };
            Cache& cache()
            {
                static Cache* c = new Cache();
                return *c;
            }

            size_t round_block(size_t bytes)
            {
                const size_t small = 512, large = size_t(2) << 20;
                if (bytes <= (size_t(1) << 20)) return (bytes + small - 1) / small * small;
                return (bytes + large - 1) / large * large;
            }

            // Takes an idle block of at least `block` bytes (at most 25% more)
            // from `pool`; returns nullptr and leaves `block` alone if none fits.
            void* take(std::multimap<size_t, void*>& pool, size_t& block)
            {
                auto it = pool.lower_bound(block);
                const size_t limit = block + (block >> 2);
                if (it == pool.end() || it->first > limit) return nullptr;
                void* p = it->second;
                block = it->first;
                pool.erase(it);
                return p;
            }
        } // namespace

        cnhip_stream_t stream() { return g_stream; }
        void set_stream(cnhip_stream_t s) { g_stream = s; }
        void synchronize() { check(cnhip_stream_synchronize(g_stream), "Device::synchronize"); }
        bool available() { return cnhip_device_count() > 0; }

        Buffer::Buffer(size_t bytes) : bytes_(bytes)
        {
            block_ = round_block(bytes == 0 ? 1 : bytes);
            Cache& c = cache();
            {
                std::lock_guard<std::mutex> lk(c.mu);
                pool_ = c.open;
                if (pool_)
                {
                    ptr_ = take(c.pools[pool_].idle, block_);
                    if (ptr_) return;
                }
                ptr_ = take(c.idle[g_stream], block_);
                if (ptr_)
                {
                    c.cached_bytes -= block_;
                    return;
                }
            }
            int st = cnhip_malloc(&ptr_, block_);
            if (st == CNHIP_ENOMEM)
            {
                empty_cache();
                st = cnhip_malloc(&ptr_, block_);
            }
            check(st, "Device::allocate");
            std::lock_guard<std::mutex> lk(c.mu);
            c.device_bytes += block_;
            c.mallocs += 1;
        }

        Buffer::~Buffer()
        {
            if (!ptr_) return;
            Cache& c = cache();
            std::lock_guard<std::mutex> lk(c.mu);
            // released during a capture: captured kernels may refer to it
            const uint64_t owner = c.open ? c.open : pool_;
            if (owner)
            {
                auto it = c.pools.find(owner);
                if (it != c.pools.end())
                {
                    it->second.idle.emplace(block_, ptr_);
                    return;
                }
            }
            c.idle[g_stream].emplace(block_, ptr_);
            c.cached_bytes += block_;
        }

        uint64_t open_pool()
        {
            Cache& c = cache();
            std::lock_guard<std::mutex> lk(c.mu);
            if (c.open) throw std::logic_error("Device::open_pool: a graph pool is already open");
            const uint64_t id = c.next_pool++;
            c.pools[id].stream = g_stream;
            c.open = id;
            return id;
        }

        void close_pool()
        {
            Cache& c = cache();
            std::lock_guard<std::mutex> lk(c.mu);
            c.open = 0;
        }

        void release_pool(uint64_t id)
        {
            Cache& c = cache();
            std::lock_guard<std::mutex> lk(c.mu);
            auto it = c.pools.find(id);
            if (it == c.pools.end()) return;
            if (c.open == id) c.open = 0;
            auto& general = c.idle[it->second.stream];
            for (auto& kv : it->second.idle)
            {
                general.emplace(kv.first, kv.second);
                c.cached_bytes += kv.first;
            }
            c.pools.erase(it);
        }

        std::shared_ptr<Buffer> allocate(size_t bytes) { return std::make_shared<Buffer>(bytes); }

        AllocatorStats allocator_stats()
        {
            Cache& c = cache();
            std::lock_guard<std::mutex> lk(c.mu);
            return AllocatorStats{c.device_bytes, c.cached_bytes, c.mallocs};
        }

        void empty_cache()
        {
            cnhip_device_synchronize();
            Cache& c = cache();
            std::lock_guard<std::mutex> lk(c.mu);
            for (auto& pool : c.idle)
                for (auto& kv : pool.second)
                {
                    cnhip_free(kv.second);
                    c.device_bytes -= kv.first;
                }
            c.idle.clear();
            c.cached_bytes = 0;
        }
    } // namespace Device

    // ---------------------------------------------------------------- DeviceTensor
    std::string shape_str(const std::vector<int64_t>& dims)
    {
        std::string s = "[";
        for (size_t i = 0; i < dims.size(); ++i)
            s += (i ? "," : "") + std::to_string(dims[i]);
        return s + "]";
    }

    static int64_t count_of(const std::vector<int64_t>& dims)
    {
        int64_t n = 1;
        for (int64_t d : dims)
        {
            if (d < 0) throw std::invalid_argument("DeviceTensor: negative dimension " + shape_str(dims));
            n *= d;
        }
        return n;
    }

    int64_t DeviceTensor::size() const { return buf_ ? count_of(dims_) : 0; }

    DeviceTensor DeviceTensor::empty(std::vector<int64_t> dims, int elem_bytes)
    {
        DeviceTensor t;
        const int64_t n = count_of(dims);
        t.dims_ = std::move(dims);
        t.buf_ = Device::allocate(static_cast<size_t>(n) * static_cast<size_t>(elem_bytes));
        t.ptr_ = t.buf_->get();
        return t;
    }

    DeviceTensor DeviceTensor::zeros(std::vector<int64_t> dims, int elem_bytes)
    {
        DeviceTensor t = empty(std::move(dims), elem_bytes);
        t.fill_zero();
        return t;
    }

    void DeviceTensor::copy_from_host(const void* src)
    {
        const size_t bytes = static_cast<size_t>(size()) * 4;
        Device::check(cnhip_memcpy_async(ptr_, src, bytes, 0, Device::stream()), "copy_from_host");
        Device::synchronize();  // src may be released by the caller right after
    }

    void DeviceTensor::copy_to_host(void* dst) const
    {
        const size_t bytes = static_cast<size_t>(size()) * 4;
        Device::check(cnhip_memcpy_async(dst, ptr_, bytes, 1, Device::stream()), "copy_to_host");
        Device::synchronize();
    }

    void DeviceTensor::copy_from_device(const DeviceTensor& src)
    {
        if (src.size() != size())
            throw std::invalid_argument("DeviceTensor::copy_from_device: size mismatch " +
                                        shape_str(src.dims()) + " vs " + shape_str(dims_));
        Device::check(cnhip_memcpy_async(ptr_, src.ptr_, static_cast<size_t>(size()) * 4, 2,
                                         Device::stream()),
                      "copy_from_device");
    }

    void DeviceTensor::fill_zero()
    {
        Device::check(cnhip_memset_async(ptr_, 0, static_cast<size_t>(size()) * 4, Device::stream()),
                      "fill_zero");
    }

    DeviceTensor DeviceTensor::view(int64_t offset, std::vector<int64_t> dims) const
    {
        const int64_t n = count_of(dims);
        if (offset < 0 || offset + n > size())
            throw std::invalid_argument("DeviceTensor::view: [" + std::to_string(offset) + ", " +
                                        std::to_string(offset + n) + ") outside " + shape_str(dims_));
        DeviceTensor t = *this;
        t.dims_ = std::move(dims);
        t.ptr_ = static_cast<char*>(ptr_) + offset * 4;
        return t;
    }

    DeviceTensor DeviceTensor::reshape(std::vector<int64_t> dims) const
    {
        if (count_of(dims) != size())
            throw std::invalid_argument("DeviceTensor::reshape: " + shape_str(dims_) + " -> " +
                                        shape_str(dims));
        DeviceTensor t = *this;
        t.dims_ = std::move(dims);
        return t;
    }
} // namespace CppNet
