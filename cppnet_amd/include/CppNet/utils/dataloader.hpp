/**
 * @file dataloader.hpp
 * @brief Mini-batch loader (ref: include/CppNet/utils/dataloader.hpp:46-109,
 *        src/CppNet/utils/dataloader.cpp:12-120).
 *
 * The reference's interface: a dataset of features [N, F] and labels [N, L]
 * (host tensors, ColMajor), batch_size, shuffle, drop_last; num_batches()
 * is N / B (drop_last) or ceil(N / B); reset() reshuffles; iterating yields
 * host Batch{features [b, F], labels [b, L]} in the epoch's index order, the
 * last batch short unless drop_last.  The shuffle is a std::shuffle of the
 * indices with a std::mt19937, seeded from Utils::set_seed's generator (the
 * reference seeds it from the clock).
 *
 * Device staging (no counterpart in the reference, whose batches are host
 * tensors that every layer call uploads):
 *  - Staging::Resident uploads the dataset once, sample-major, and assembles
 *    each batch in HBM with one gather kernel over the epoch's indices
 *    (cnhip_gather_batch): no host work and no PCIe traffic per batch.  For
 *    datasets that fit the GPU's memory, which on a 288 GB MI355X is most.
 *  - Staging::Stream keeps the dataset on the host: a worker thread gathers
 *    the next batches (with up to 8 helper threads for large ones) into four
 *    page-locked buffers, round robin, and uploads each on its own stream
 *    while the GPU runs the current step; the consuming stream waits on the
 *    upload's event, and the upload of batch k+4 into a slot waits on the
 *    event of batch k's consumption.  Both streams keep the default priority.
 * next_device() / next_into() deliver the epoch's next batch on
 * Device::stream() with the same values, in the same order, as the host
 * iterator.
 */
#ifndef CPPNET_UTILS_DATALOADER_HPP
#define CPPNET_UTILS_DATALOADER_HPP

#include <cstddef>
#include <cstdint>
#include <memory>
#include <random>
#include <vector>

#include "CppNet/core/tensor.hpp"

namespace CppNet
{
    namespace Utils
    {
        struct Batch
        {
            Tensor<float, 2> features;  ///< [batch, F]
            Tensor<float, 2> labels;    ///< [batch, L]
        };

        struct DeviceBatch
        {
            DeviceTensor features;  ///< [batch, F], HBM
            DeviceTensor labels;    ///< [batch, L], HBM
        };

        enum class Staging
        {
            Resident = 1,
            Stream = 2
        };

        class DataLoader
        {
        public:
            /// The dataset is taken by value: pass rvalues to move it in
            /// instead of holding a second host copy.
            DataLoader(Tensor<float, 2> features, Tensor<float, 2> labels, int batch_size, bool shuffle = true,
                       bool drop_last = false);
            ~DataLoader();
            DataLoader(const DataLoader&) = delete;
            DataLoader& operator=(const DataLoader&) = delete;

            /// Reshuffles (when shuffling) and restarts the device epoch.
            void reset();
            std::size_t num_batches() const { return num_batches_; }
            int num_samples() const { return num_samples_; }
            int get_batch_size() const { return batch_size_; }

            class Iterator
            {
            public:
                Iterator(DataLoader* loader, std::size_t batch_idx) : loader_(loader), batch_idx_(batch_idx) {}
                Batch operator*() const { return loader_->get_batch(batch_idx_); }
                Iterator& operator++()
                {
                    ++batch_idx_;
                    return *this;
                }
                bool operator!=(const Iterator& other) const { return batch_idx_ != other.batch_idx_; }

            private:
                DataLoader* loader_;
                std::size_t batch_idx_;
            };
            Iterator begin() { return Iterator(this, 0); }
            Iterator end() { return Iterator(this, num_batches_); }

            /// Batch k of the current epoch on the host (the reference's get_batch).
            Batch get_batch(std::size_t batch_idx) const;
            /// The current epoch's sample order.
            const std::vector<int>& indices() const { return indices_; }
            /// Re-seeds the shuffle generator and reshuffles.
            void set_seed(uint64_t seed);

            /// Chooses the device staging and restarts the device epoch.
            void to_device(Staging mode);
            /// Size of the epoch's next batch (0 at the end of the epoch).
            int64_t next_size() const;
            /// The epoch's next batch in new device tensors; false at the end of the epoch.
            bool next_device(DeviceBatch& out);
            /// The epoch's next batch into existing device buffers of at least
            /// [batch, F] / [batch, L] floats; returns its size (0 at the end).
            int64_t next_into(float* features, float* labels);

        private:
            struct Stager;
            void restart_device();
            void gather_host(std::size_t batch_idx, float* x, float* y, int threads) const;

            Tensor<float, 2> features_, labels_;
            int batch_size_;
            bool shuffle_, drop_last_;
            int num_samples_, num_features_, num_labels_;
            std::size_t num_batches_;
            std::vector<int> indices_;
            std::mt19937 gen_;
            std::unique_ptr<Stager> stager_;
        };
    } // namespace Utils
} // namespace CppNet

#endif
