// DataLoader with device staging (ref: src/CppNet/utils/dataloader.cpp:12-120).
#include "CppNet/utils/dataloader.hpp"

#include <algorithm>
#include <condition_variable>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "CppNet/core/device.hpp"
#include "CppNet/utils/init.hpp"

namespace CppNet
{
    namespace Utils
    {
        struct DataLoader::Stager
        {
            Staging mode;
            int device = 0;
            std::size_t cursor = 0;  // next batch of the epoch to deliver

            // Resident: the dataset sample-major in HBM and the epoch's order.
            // The gathers run asynchronously on the consumer's stream, so the
            // order is double-buffered (epoch e reads idx[e % 2]) and each
            // buffer is fenced: after every gather that reads idx[p], an event
            // per consumer stream is re-recorded, and the host waits on
            // buffer p's events before it overwrites idx[p] two epochs later
            // (long complete by then) or frees the dataset.
            DeviceTensor xs, ys, idx[2];
            int cur = 0;
            std::vector<std::pair<cnhip_stream_t, void*>> fence[2];

            void fence_read(cnhip_stream_t s)
            {
                void* ev = nullptr;
                for (auto& f : fence[cur])
                    if (f.first == s) ev = f.second;
                if (!ev)
                {
                    Device::check(cnhip_event_create(&ev), "DataLoader::next");
                    fence[cur].emplace_back(s, ev);
                }
                Device::check(cnhip_event_record(ev, s), "DataLoader::next");
            }
            void wait_fences(int p)
            {
                for (auto& f : fence[p])
                {
                    (void)cnhip_event_synchronize(f.second);
                    (void)cnhip_event_destroy(f.second);
                }
                fence[p].clear();
            }

            // Stream: kSlots page-locked host slots and as many device slots,
            // each [B*F features | B*L labels]; batch k uses slot k % kSlots.
            // copied[s] marks the end of a slot's upload (copy stream),
            // consumed[s] the end of its hand-over to the consumer (consumer's
            // stream).  The worker runs at most kSlots batches ahead.
            static constexpr int kSlots = 4;
            cnhip_stream_t copy = nullptr;
            void* copied[kSlots] = {};
            void* consumed[kSlots] = {};
            bool copied_rec[kSlots] = {}, consumed_rec[kSlots] = {};
            float* pin[kSlots] = {};
            DeviceTensor slot[kSlots];
            std::thread worker;
            std::mutex mu;
            std::condition_variable cv;
            std::size_t produced = 0, taken = 0;
            bool stop = false;
            std::string error;

            ~Stager()
            {
                stop_worker();
                wait_fences(0);  // gathers still queued read xs, ys and idx
                wait_fences(1);
                if (copy) (void)cnhip_stream_synchronize(copy);
                for (int s = 0; s < kSlots; ++s)
                {
                    // the consumer's copies out of the device slots must be done
                    if (consumed_rec[s]) (void)cnhip_event_synchronize(consumed[s]);
                    (void)cnhip_host_free(pin[s]);
                    (void)cnhip_event_destroy(copied[s]);
                    (void)cnhip_event_destroy(consumed[s]);
                }
                if (copy) (void)cnhip_stream_destroy(copy);
            }

            void stop_worker()
            {
                {
                    std::lock_guard<std::mutex> lk(mu);
                    stop = true;
                }
                cv.notify_all();
                if (worker.joinable()) worker.join();
            }
        };

        DataLoader::DataLoader(Tensor<float, 2> features, Tensor<float, 2> labels, int batch_size, bool shuffle,
                               bool drop_last)
            : features_(std::move(features)), labels_(std::move(labels)), batch_size_(batch_size), shuffle_(shuffle),
              drop_last_(drop_last), gen_(static_cast<std::mt19937::result_type>(next_seed()))
        {
            num_samples_ = static_cast<int>(features_.dimension(0));
            num_features_ = static_cast<int>(features_.dimension(1));
            num_labels_ = static_cast<int>(labels_.dimension(1));
            // dataloader.cpp:22-28
            if (labels_.dimension(0) != num_samples_)
                throw std::invalid_argument("DataLoader: features and labels must have the same number of samples");
            if (batch_size_ <= 0) throw std::invalid_argument("DataLoader: batch_size must be > 0");
            num_batches_ = drop_last_ ? static_cast<std::size_t>(num_samples_ / batch_size_)
                                      : static_cast<std::size_t>((num_samples_ + batch_size_ - 1) / batch_size_);
            indices_.resize(static_cast<std::size_t>(num_samples_));
            for (int i = 0; i < num_samples_; ++i) indices_[static_cast<std::size_t>(i)] = i;
            if (shuffle_) std::shuffle(indices_.begin(), indices_.end(), gen_);
        }

        DataLoader::~DataLoader() = default;

        void DataLoader::reset()
        {
            if (stager_) stager_->stop_worker();  // it reads indices_
            if (shuffle_) std::shuffle(indices_.begin(), indices_.end(), gen_);
            if (stager_) restart_device();
        }

        void DataLoader::set_seed(uint64_t seed)
        {
            gen_.seed(static_cast<std::mt19937::result_type>(seed));
            for (int i = 0; i < num_samples_; ++i) indices_[static_cast<std::size_t>(i)] = i;
            if (stager_) stager_->stop_worker();
            if (shuffle_) std::shuffle(indices_.begin(), indices_.end(), gen_);
            if (stager_) restart_device();
        }

        // dataloader.cpp:68-88, written ColMajor [b, F] / [b, L]: column by
        // column (each column of the dataset is contiguous), the columns split
        // over `threads` host threads
        void DataLoader::gather_host(std::size_t k, float* x, float* y, int threads) const
        {
            const int64_t start = static_cast<int64_t>(k) * batch_size_;
            const int64_t bs = std::min<int64_t>(batch_size_, num_samples_ - start);
            const int64_t N = num_samples_, F = num_features_, C = num_features_ + num_labels_;
            const int* rows = indices_.data() + start;
            auto columns = [&](int64_t c0, int64_t c1) {
                for (int64_t c = c0; c < c1; ++c)
                {
                    const float* col = c < F ? features_.data() + N * c : labels_.data() + N * (c - F);
                    float* out = c < F ? x + bs * c : y + bs * (c - F);
                    for (int64_t i = 0; i < bs; ++i) out[i] = col[rows[i]];
                }
            };
            const int T = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(threads, C)));
            if (T == 1)
            {
                columns(0, C);
                return;
            }
            std::vector<std::thread> pool;
            for (int t = 1; t < T; ++t) pool.emplace_back(columns, C * t / T, C * (t + 1) / T);
            columns(0, C / T);
            for (auto& th : pool) th.join();
        }

        Batch DataLoader::get_batch(std::size_t k) const
        {
            if (k >= num_batches_) throw std::out_of_range("DataLoader: batch index out of range");
            const int64_t bs = std::min<int64_t>(batch_size_, num_samples_ - static_cast<int64_t>(k) * batch_size_);
            Batch b;
            b.features = Tensor<float, 2>(bs, static_cast<int64_t>(num_features_));
            b.labels = Tensor<float, 2>(bs, static_cast<int64_t>(num_labels_));
            gather_host(k, b.features.data(), b.labels.data(), 1);
            return b;
        }

        void DataLoader::to_device(Staging mode)
        {
            if (mode != Staging::Resident && mode != Staging::Stream)
                throw std::invalid_argument("DataLoader::to_device: unknown staging mode");
            stager_.reset();
            auto st = std::make_unique<Stager>();
            st->mode = mode;
            Device::check(cnhip_get_device(&st->device), "DataLoader::to_device");
            const int64_t N = num_samples_, F = num_features_, L = num_labels_, B = batch_size_;
            if (mode == Staging::Resident)
            {
                // upload once, then lay samples out contiguously: [N, F] -> [F, N]
                DeviceTensor tx = DeviceTensor::from_host(features_);
                DeviceTensor ty = DeviceTensor::from_host(labels_);
                st->xs = DeviceTensor::empty({F, N});
                st->ys = DeviceTensor::empty({L, N});
                Device::check(cnhip_transpose(tx.data(), st->xs.data(), N, F, Device::stream()), "DataLoader");
                Device::check(cnhip_transpose(ty.data(), st->ys.data(), N, L, Device::stream()), "DataLoader");
                st->idx[0] = DeviceTensor::empty({N});
                st->idx[1] = DeviceTensor::empty({N});
                Device::synchronize();
            }
            else
            {
                Device::check(cnhip_stream_create(&st->copy), "DataLoader::to_device");
                const std::size_t floats = static_cast<std::size_t>(B * (F + L));
                for (int s = 0; s < Stager::kSlots; ++s)
                {
                    Device::check(cnhip_event_create(&st->copied[s]), "DataLoader::to_device");
                    Device::check(cnhip_event_create(&st->consumed[s]), "DataLoader::to_device");
                    void* p = nullptr;
                    Device::check(cnhip_host_alloc(&p, floats * 4), "DataLoader::to_device");
                    st->pin[s] = static_cast<float*>(p);
                    st->slot[s] = DeviceTensor::empty({static_cast<int64_t>(floats)});
                }
            }
            stager_ = std::move(st);
            restart_device();
        }

        void DataLoader::restart_device()
        {
            Stager& st = *stager_;
            st.cursor = 0;
            if (st.mode == Staging::Resident)
            {
                st.cur ^= 1;
                st.wait_fences(st.cur);  // the epoch before last has finished reading it
                if (num_samples_) st.idx[st.cur].copy_from_host(indices_.data());  // one small upload per epoch
                return;
            }
            st.stop_worker();
            st.stop = false;
            st.produced = st.taken = 0;
            st.error.clear();
            // the worker is bound to this Stager, not to stager_: to_device()
            // empties stager_ before the old Stager's destructor joins it
            Stager* self = &st;
            st.worker = std::thread([this, self] {
                Stager& s = *self;
                try
                {
                    Device::check(cnhip_set_device(s.device), "DataLoader worker");
                    const int64_t F = num_features_, L = num_labels_, B = batch_size_;
                    // one gather thread per 64 Ki values of a batch, at most 8
                    // and at most half the host's hardware threads
                    const int64_t hw = std::max<int64_t>(1, std::thread::hardware_concurrency() / 2);
                    const int threads =
                        static_cast<int>(std::max<int64_t>(1, std::min<int64_t>({(B * (F + L)) >> 16, 8, hw})));
                    for (std::size_t k = 0; k < num_batches_; ++k)
                    {
                        {
                            std::unique_lock<std::mutex> lk(s.mu);
                            s.cv.wait(lk, [&] { return s.stop || k < s.taken + Stager::kSlots; });
                            if (s.stop) return;
                        }
                        const int j = static_cast<int>(k % Stager::kSlots);
                        const int64_t start = static_cast<int64_t>(k) * B;
                        const int64_t bs = std::min<int64_t>(B, num_samples_ - start);
                        // the slot's previous upload has finished reading the host buffer
                        if (s.copied_rec[j]) Device::check(cnhip_event_synchronize(s.copied[j]), "DataLoader worker");
                        gather_host(k, s.pin[j], s.pin[j] + B * F, threads);
                        // and its previous contents have been handed over on the device
                        if (s.consumed_rec[j])
                            Device::check(cnhip_stream_wait_event(s.copy, s.consumed[j]), "DataLoader worker");
                        float* d = s.slot[j].data();
                        Device::check(cnhip_memcpy_async(d, s.pin[j], static_cast<size_t>(bs * F) * 4, 0, s.copy),
                                      "DataLoader worker");
                        Device::check(cnhip_memcpy_async(d + B * F, s.pin[j] + B * F, static_cast<size_t>(bs * L) * 4,
                                                         0, s.copy),
                                      "DataLoader worker");
                        Device::check(cnhip_event_record(s.copied[j], s.copy), "DataLoader worker");
                        {
                            std::lock_guard<std::mutex> lk(s.mu);
                            s.copied_rec[j] = true;
                            s.produced = k + 1;
                        }
                        s.cv.notify_all();
                    }
                }
                catch (const std::exception& e)
                {
                    std::lock_guard<std::mutex> lk(s.mu);
                    s.error = e.what();
                    s.cv.notify_all();
                }
            });
        }

        int64_t DataLoader::next_size() const
        {
            if (!stager_) throw std::logic_error("DataLoader: call to_device() first");
            const std::size_t k = stager_->cursor;
            if (k >= num_batches_) return 0;
            return std::min<int64_t>(batch_size_, num_samples_ - static_cast<int64_t>(k) * batch_size_);
        }

        int64_t DataLoader::next_into(float* x, float* y)
        {
            const int64_t bs = next_size();
            if (bs == 0) return 0;
            if (!x || !y) throw std::invalid_argument("DataLoader::next_into: NULL buffer");
            Stager& st = *stager_;
            const std::size_t k = st.cursor;
            const int64_t N = num_samples_, F = num_features_, L = num_labels_, B = batch_size_;
            if (st.mode == Staging::Resident)
            {
                const int32_t* idx = st.idx[st.cur].idata() + static_cast<int64_t>(k) * B;
                Device::check(cnhip_gather_batch(st.xs.data(), st.ys.data(), idx, x, y, N, F, L, bs, Device::stream()),
                              "DataLoader::next");
                st.fence_read(Device::stream());
            }
            else
            {
                {
                    std::unique_lock<std::mutex> lk(st.mu);
                    st.cv.wait(lk, [&] { return st.produced > k || !st.error.empty(); });
                    if (st.produced <= k) throw std::runtime_error("DataLoader staging failed: " + st.error);
                }
                const int j = static_cast<int>(k % Stager::kSlots);
                Device::check(cnhip_stream_wait_event(Device::stream(), st.copied[j]), "DataLoader::next");
                const float* d = st.slot[j].data();
                Device::check(cnhip_memcpy_async(x, d, static_cast<size_t>(bs * F) * 4, 2, Device::stream()),
                              "DataLoader::next");
                Device::check(cnhip_memcpy_async(y, d + B * F, static_cast<size_t>(bs * L) * 4, 2, Device::stream()),
                              "DataLoader::next");
                Device::check(cnhip_event_record(st.consumed[j], Device::stream()), "DataLoader::next");
                {
                    std::lock_guard<std::mutex> lk(st.mu);
                    st.consumed_rec[j] = true;
                    st.taken = k + 1;
                }
                st.cv.notify_all();
            }
            st.cursor = k + 1;
            return bs;
        }

        bool DataLoader::next_device(DeviceBatch& out)
        {
            const int64_t bs = next_size();
            if (bs == 0) return false;
            out.features = DeviceTensor::empty({bs, static_cast<int64_t>(num_features_)});
            out.labels = DeviceTensor::empty({bs, static_cast<int64_t>(num_labels_)});
            next_into(out.features.data(), out.labels.data());
            return true;
        }
    } // namespace Utils
} // namespace CppNet
