// Embedding / MultiHeadAttention / BatchNorm / MeanPool1D / Residual / GELU
// on device "gpu" (ref: src/CppNet/layers/embedding.cpp:33-185,
// attention.cpp:35-587, batch_norm.cpp:25-401, mean_pool1d.cpp:24-150,
// residual.cpp:23-159; GELU has no reference).
#include <cmath>
#include <stdexcept>
#include <string>
#include <vector>

#include "CppNet/activations/gelu.hpp"
#include "CppNet/layers/attention.hpp"
#include "CppNet/layers/batch_norm.hpp"
#include "CppNet/layers/embedding.hpp"
#include "CppNet/layers/mean_pool1d.hpp"
#include "CppNet/layers/residual.hpp"
#include "CppNet/optimizers/optimizer.hpp"
#include "CppNet/utils/init.hpp"

namespace CppNet
{
    namespace Layers
    {
        namespace
        {
            int check_rows(int rows, const char* who)
            {
                if (rows != CNHIP_ROWS_REF && rows != CNHIP_ROWS_BY_SAMPLE)
                    throw std::invalid_argument(std::string(who) + ": row order must be 0 or 1");
                return rows;
            }
            // host tensors always carry the reference's row order
            void require_ref_rows(int rows, const char* who)
            {
                if (rows != CNHIP_ROWS_REF)
                    throw std::logic_error(std::string(who) +
                                           ": host tensors are in the reference row order; this layer runs by sample");
            }

            void check_2d(const Tensor<float, 2>& t, int64_t r, int64_t c, const char* who)
            {
                if (t.dimension(0) != r || t.dimension(1) != c)
                    throw std::invalid_argument(std::string(who) + ": expected [" + std::to_string(r) + ", " +
                                                std::to_string(c) + "]");
            }
        } // namespace

        // ---------------------------------------------------------------- Embedding
        Embedding::Embedding(int vocab_size, int embed_dim, const std::string& device)
            : vocab_size_(vocab_size), embed_dim_(embed_dim), device_(device)
        {
            if (vocab_size <= 0 || embed_dim <= 0)
                throw std::invalid_argument("Embedding: vocab_size and embed_dim must be positive");
            require_gpu_device(device_, "Embedding");
            Wt_ = DeviceTensor::empty({embed_dim_, vocab_size_});
            gWt_ = DeviceTensor::empty({embed_dim_, vocab_size_});
            oob_ = DeviceTensor::zeros({1});
            // U(-1/sqrt(D), 1/sqrt(D)) (embedding.cpp:38-39)
            const float scale = 1.0f / std::sqrt(static_cast<float>(embed_dim_));
            set_weight(Utils::uniform_init(vocab_size_, embed_dim_, -scale, scale));
        }

        DeviceTensor Embedding::forward(const DeviceTensor& ids) { return forward(ids, false); }

        DeviceTensor Embedding::forward(const DeviceTensor& ids, bool ids_checked)
        {
            if (ids.rank() != 2) throw std::runtime_error("Embedding::forward: expected ids [B, S]");
            const int64_t B = ids.dimension(0), S = ids.dimension(1);
            DeviceTensor out = DeviceTensor::empty({B, S, embed_dim_});
            if (!ids_checked) oob_.fill_zero();
            Device::check(cnhip_embedding_forward_rows(ids.idata(), Wt_.data(), out.data(), B, S, vocab_size_,
                                                       embed_dim_, ids_checked ? nullptr : oob_.idata(), rows_,
                                                       Device::stream()),
                          "Embedding::forward");
            if (ids_checked)
            {
                ids_cache_ = ids;
                return out;
            }
            int32_t bad = 0;
            oob_.copy_to_host(&bad);
            if (bad > 0)
            {
                // error path: name the first offending id in (n, s) order (embedding.cpp:87-90)
                std::vector<int32_t> h(static_cast<size_t>(B * S));
                ids.copy_to_host(h.data());
                for (int64_t n = 0; n < B; ++n)
                    for (int64_t s = 0; s < S; ++s)
                    {
                        const int32_t id = h[static_cast<size_t>(n + B * s)];
                        if (id < 0 || id >= vocab_size_)
                            throw std::out_of_range("Embedding: token ID " + std::to_string(id) +
                                                    " out of range [0, " + std::to_string(vocab_size_) + ")");
                    }
            }
            ids_cache_ = ids;
            return out;
        }

        DeviceTensor Embedding::backward(const DeviceTensor& g) { return backward(g, true); }

        DeviceTensor Embedding::backward(const DeviceTensor& g, bool input_grad)
        {
            if (!ids_cache_.defined()) throw std::runtime_error("Embedding::backward before forward");
            const int64_t B = ids_cache_.dimension(0), S = ids_cache_.dimension(1);
            if (g.rank() != 3 || g.dimension(0) != B || g.dimension(1) != S || g.dimension(2) != embed_dim_)
                throw std::runtime_error("Embedding::backward: grad shape " + shape_str(g.dims()));
            Device::check(cnhip_embedding_backward_rows(ids_cache_.idata(), g.data(), gWt_.data(), B, S,
                                                        vocab_size_, embed_dim_, rows_, Device::stream()),
                          "Embedding::backward");
            grads_zero_ = false;
            return input_grad ? DeviceTensor::zeros({B, S, embed_dim_}) : DeviceTensor();  // embedding.cpp:171-174
        }

        Tensor<float, 3> Embedding::forward(const Tensor<int, 2>& input)
        {
            require_ref_rows(rows_, "Embedding::forward");
            return forward(DeviceTensor::from_host(input)).to_host<float, 3>();
        }
        Tensor<float, 3> Embedding::backward(const Tensor<float, 3>& g)
        {
            require_ref_rows(rows_, "Embedding::backward");
            return backward(DeviceTensor::from_host(g)).to_host<float, 3>();
        }

        void Embedding::set_row_order(int rows) { rows_ = check_rows(rows, "Embedding::set_row_order"); }

        void Embedding::materialize_grads() const
        {
            if (!grads_zero_) return;
            auto* self = const_cast<Embedding*>(this);
            self->gWt_.fill_zero();
            self->grads_zero_ = false;
        }

        void Embedding::step(Optimizers::Optimizer& optimizer, float learning_rate)
        {
            if (!trainable_) return;
            materialize_grads();
            optimizer.update(Wt_.data(), gWt_.data(), Wt_.size(), learning_rate);
            grads_zero_ = true;  // embedding.cpp:184
        }

        namespace
        {
            // token-major [D, V] <-> reference ColMajor [V, D] through a device transpose
            Tensor<float, 2> table_to_host(const DeviceTensor& t, int64_t V, int64_t D)
            {
                DeviceTensor tmp = DeviceTensor::empty({V, D});
                Device::check(cnhip_transpose(t.data(), tmp.data(), D, V, Device::stream()), "Embedding");
                return tmp.to_host<float, 2>();
            }
        } // namespace

        const Tensor<float, 2> Embedding::get_weight() const { return table_to_host(Wt_, vocab_size_, embed_dim_); }
        const Tensor<float, 2> Embedding::get_grad_weight() const
        {
            materialize_grads();
            return table_to_host(gWt_, vocab_size_, embed_dim_);
        }
        void Embedding::set_weight(const Tensor<float, 2>& w)
        {
            check_2d(w, vocab_size_, embed_dim_, "Embedding::set_weight");
            DeviceTensor tmp = DeviceTensor::from_host(w);
            Device::check(cnhip_transpose(tmp.data(), Wt_.data(), vocab_size_, embed_dim_, Device::stream()),
                          "Embedding::set_weight");
            Device::synchronize();  // tmp is released on return
        }

        // ---------------------------------------------------------------- MultiHeadAttention
        MultiHeadAttention::MultiHeadAttention(int embed_dim, int num_heads, const std::string& device)
            : embed_dim_(embed_dim), num_heads_(num_heads), device_(device)
        {
            if (embed_dim <= 0 || num_heads <= 0)
                throw std::invalid_argument("embed_dim and num_heads must be positive");
            if (embed_dim_ % num_heads_ != 0)
                throw std::invalid_argument("embed_dim must be divisible by num_heads");  // attention.cpp:39-43
            require_gpu_device(device_, "MultiHeadAttention");
            const int64_t D = embed_dim_;
            Wall_ = DeviceTensor::empty({D, 4 * D});
            gWall_ = DeviceTensor::empty({D, 4 * D});
            for (int i = 0; i < 4; ++i)
            {
                W_[i] = Wall_.view(i * D * D, {D, D});
                gW_[i] = gWall_.view(i * D * D, {D, D});
            }
            for (int i = 0; i < 4; ++i)  // attention.cpp:47-50, in the order q, k, v, o
                set_weight(i, Utils::xavier_uniform(embed_dim_, embed_dim_));
        }

        DeviceTensor& MultiHeadAttention::weight(int which)
        {
            if (which < 0 || which > 3) throw std::out_of_range("MultiHeadAttention: weight index");
            return W_[which];
        }
        DeviceTensor& MultiHeadAttention::grad_weight(int which)
        {
            if (which < 0 || which > 3) throw std::out_of_range("MultiHeadAttention: weight index");
            materialize_grads();
            return gW_[which];
        }

        DeviceTensor MultiHeadAttention::forward(const DeviceTensor& q, const DeviceTensor& k, const DeviceTensor& v)
        {
            return forward_residual(q, k, v, DeviceTensor());
        }

        DeviceTensor MultiHeadAttention::forward_residual(const DeviceTensor& q, const DeviceTensor& k,
                                                          const DeviceTensor& v, const DeviceTensor& residual)
        {
            for (const DeviceTensor* t : {&q, &k, &v})
                if (t->rank() != 3 || t->dimension(2) != embed_dim_ || t->dims() != q.dims())
                    throw std::runtime_error("MultiHeadAttention::forward: expected query/key/value [B, S, " +
                                             std::to_string(embed_dim_) + "] of one shape");
            if (residual.defined() && residual.size() != q.size())
                throw std::runtime_error("MultiHeadAttention::forward_residual: residual shape " +
                                         shape_str(residual.dims()));
            const int64_t B = q.dimension(0), S = q.dimension(1), D = embed_dim_;
            cache_ = DeviceTensor::empty({cnhip_mha_cache_floats(B, S, D)});
            DeviceTensor out = DeviceTensor::empty({B, S, D});
            Device::check(cnhip_mha_forward_rows(q.data(), k.data(), v.data(), W_[0].data(), W_[1].data(),
                                                 W_[2].data(), W_[3].data(),
                                                 residual.defined() ? residual.data() : nullptr, out.data(),
                                                 cache_.data(), B, S, D, num_heads_, rows_, Device::stream()),
                          "MultiHeadAttention::forward");
            q_cache_ = q;
            k_cache_ = k;
            v_cache_ = v;
            return out;
        }

        DeviceTensor MultiHeadAttention::backward(const DeviceTensor& g) { return backward_residual(g, DeviceTensor()); }

        DeviceTensor MultiHeadAttention::backward_residual(const DeviceTensor& g, const DeviceTensor& skip_grad)
        {
            if (!cache_.defined()) throw std::runtime_error("MultiHeadAttention::backward before forward");
            if (g.dims() != q_cache_.dims())
                throw std::runtime_error("MultiHeadAttention::backward: grad shape " + shape_str(g.dims()));
            if (skip_grad.defined() && skip_grad.size() != g.size())
                throw std::runtime_error("MultiHeadAttention::backward_residual: skip gradient shape " +
                                         shape_str(skip_grad.dims()));
            const int64_t B = g.dimension(0), S = g.dimension(1), D = embed_dim_;
            DeviceTensor dx = DeviceTensor::empty({B, S, D});
            Device::check(cnhip_mha_backward_rows(
                              q_cache_.data(), k_cache_.data(), v_cache_.data(), W_[0].data(), W_[1].data(),
                              W_[2].data(), W_[3].data(), cache_.data(), g.data(),
                              skip_grad.defined() ? skip_grad.data() : nullptr, gW_[0].data(), gW_[1].data(),
                              gW_[2].data(), gW_[3].data(), dx.data(), B, S, D, num_heads_, rows_,
                              Device::stream()),
                          "MultiHeadAttention::backward");
            grads_zero_ = false;
            return dx;
        }

        Tensor<float, 3> MultiHeadAttention::forward(const Tensor<float, 3>& q, const Tensor<float, 3>& k,
                                                     const Tensor<float, 3>& v)
        {
            require_ref_rows(rows_, "MultiHeadAttention::forward");
            DeviceTensor dq = DeviceTensor::from_host(q);
            if (&k == &q && &v == &q) return forward(dq, dq, dq).to_host<float, 3>();
            return forward(dq, DeviceTensor::from_host(k), DeviceTensor::from_host(v)).to_host<float, 3>();
        }
        Tensor<float, 3> MultiHeadAttention::backward(const Tensor<float, 3>& g)
        {
            require_ref_rows(rows_, "MultiHeadAttention::backward");
            return backward(DeviceTensor::from_host(g)).to_host<float, 3>();
        }

        void MultiHeadAttention::set_row_order(int rows)
        {
            rows_ = check_rows(rows, "MultiHeadAttention::set_row_order");
        }

        void MultiHeadAttention::materialize_grads() const
        {
            if (!grads_zero_) return;
            auto* self = const_cast<MultiHeadAttention*>(this);
            self->gWall_.fill_zero();
            self->grads_zero_ = false;
        }

        void MultiHeadAttention::step(Optimizers::Optimizer& optimizer, float learning_rate)
        {
            if (!trainable_) return;
            materialize_grads();
            for (int i = 0; i < 4; ++i)  // attention.cpp:578-581
                optimizer.update(W_[i].data(), gW_[i].data(), W_[i].size(), learning_rate);
            grads_zero_ = true;  // attention.cpp:583-586
        }

        const Tensor<float, 2> MultiHeadAttention::get_weight(int which) const
        {
            if (which < 0 || which > 3) throw std::out_of_range("MultiHeadAttention: weight index");
            return W_[which].to_host<float, 2>();
        }
        const Tensor<float, 2> MultiHeadAttention::get_grad_weight(int which) const
        {
            if (which < 0 || which > 3) throw std::out_of_range("MultiHeadAttention: weight index");
            materialize_grads();
            return gW_[which].to_host<float, 2>();
        }
        void MultiHeadAttention::set_weight(int which, const Tensor<float, 2>& w)
        {
            if (which < 0 || which > 3) throw std::out_of_range("MultiHeadAttention: weight index");
            check_2d(w, embed_dim_, embed_dim_, "MultiHeadAttention::set_weight");
            W_[which].copy_from_host(w.data());
        }
        const Tensor<float, 3> MultiHeadAttention::get_attention_weights() const
        {
            if (!cache_.defined()) throw std::runtime_error("MultiHeadAttention: no forward yet");
            const int64_t B = q_cache_.dimension(0), S = q_cache_.dimension(1), D = embed_dim_;
            // the cache holds A^T per sample: A[b][i][j] at 3BSD + b*S*S + j + S*i
            std::vector<float> at(static_cast<size_t>(B * S * S));
            cache_.view(3 * B * S * D, {B * S * S}).copy_to_host(at.data());
            Tensor<float, 3> A(B, S, S);
            for (int64_t b = 0; b < B; ++b)
                for (int64_t i = 0; i < S; ++i)
                    for (int64_t j = 0; j < S; ++j) A(b, i, j) = at[static_cast<size_t>(b * S * S + j + S * i)];
            return A;
        }

        // ---------------------------------------------------------------- BatchNorm
        BatchNorm::BatchNorm(int num_features, float momentum, float eps, const std::string& device)
            : num_features_(num_features), momentum_(momentum), eps_(eps), device_(device)
        {
            if (num_features <= 0) throw std::invalid_argument("BatchNorm: num_features must be positive");
            require_gpu_device(device_, "BatchNorm");
            const int64_t F = num_features_;
            Tensor<float, 1> ones(F);
            ones.setConstant(1.0f);
            gamma_ = DeviceTensor::from_host(ones);  // batch_norm.cpp:30-33
            beta_ = DeviceTensor::zeros({F});
            rmean_ = DeviceTensor::zeros({F});
            rvar_ = DeviceTensor::from_host(ones);  // batch_norm.cpp:40-43
            bmean_ = DeviceTensor::zeros({F});
            bvar_ = DeviceTensor::zeros({F});
            ggamma_ = DeviceTensor::empty({F});
            gbeta_ = DeviceTensor::empty({F});
        }

        DeviceTensor BatchNorm::forward(const DeviceTensor& x)
        {
            if (x.rank() != 2 || x.dimension(1) != num_features_)
                throw std::runtime_error("BatchNorm: input features (" +
                                         std::to_string(x.rank() == 2 ? x.dimension(1) : -1) +
                                         ") != num_features (" + std::to_string(num_features_) + ")");
            const int64_t N = x.dimension(0), F = num_features_;
            DeviceTensor y = DeviceTensor::empty({N, F});
            // training: the backward recomputes xhat from x and the batch
            // statistics (bit for bit), so it is not stored; eval: the
            // backward reads the cached xhat, as the reference's does
            xhat_ = training_ ? DeviceTensor() : DeviceTensor::empty({N, F});
            if (training_)
                Device::check(cnhip_batchnorm_forward(x.data(), y.data(), nullptr, gamma_.data(), beta_.data(),
                                                      rmean_.data(), rvar_.data(), bmean_.data(), bvar_.data(), N, F,
                                                      momentum_, eps_, Device::stream()),
                              "BatchNorm::forward");
            else
                Device::check(cnhip_batchnorm_forward_eval(x.data(), y.data(), xhat_.data(), gamma_.data(),
                                                           beta_.data(), rmean_.data(), rvar_.data(), N, F, eps_,
                                                           Device::stream()),
                              "BatchNorm::forward");
            in_cache_ = x;
            return y;
        }

        DeviceTensor BatchNorm::backward(const DeviceTensor& g)
        {
            if (!in_cache_.defined()) throw std::runtime_error("BatchNorm::backward before forward");
            if (g.dims() != in_cache_.dims())
                throw std::runtime_error("BatchNorm::backward: grad shape " + shape_str(g.dims()));
            const int64_t N = g.dimension(0), F = num_features_;
            DeviceTensor dx = DeviceTensor::empty({N, F});
            Device::check(cnhip_batchnorm_backward(g.data(), in_cache_.data(),
                                                   xhat_.defined() ? xhat_.data() : nullptr, gamma_.data(),
                                                   bmean_.data(), bvar_.data(), ggamma_.data(), gbeta_.data(),
                                                   dx.data(), N, F, eps_, Device::stream()),
                          "BatchNorm::backward");
            grads_zero_ = false;
            return dx;
        }

        Tensor<float, 2> BatchNorm::forward(const Tensor<float, 2>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 2>();
        }
        Tensor<float, 2> BatchNorm::backward(const Tensor<float, 2>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 2>();
        }

        void BatchNorm::materialize_grads() const
        {
            if (!grads_zero_) return;
            auto* self = const_cast<BatchNorm*>(this);
            self->ggamma_.fill_zero();
            self->gbeta_.fill_zero();
            self->grads_zero_ = false;
        }

        void BatchNorm::step(Optimizers::Optimizer& optimizer, float learning_rate)
        {
            if (!trainable_) return;
            materialize_grads();
            optimizer.update(gamma_.data(), ggamma_.data(), gamma_.size(), learning_rate);
            optimizer.update(beta_.data(), gbeta_.data(), beta_.size(), learning_rate);
            grads_zero_ = true;  // batch_norm.cpp:399-400
        }

        const Tensor<float, 1> BatchNorm::get_grad_gamma() const
        {
            materialize_grads();
            return ggamma_.to_host<float, 1>();
        }
        const Tensor<float, 1> BatchNorm::get_grad_beta() const
        {
            materialize_grads();
            return gbeta_.to_host<float, 1>();
        }
        namespace
        {
            void set_vec(DeviceTensor& t, const Tensor<float, 1>& v, const char* who)
            {
                if (v.dimension(0) != t.size()) throw std::invalid_argument(std::string(who) + ": size mismatch");
                t.copy_from_host(v.data());
            }
        } // namespace
        void BatchNorm::set_gamma(const Tensor<float, 1>& g) { set_vec(gamma_, g, "BatchNorm::set_gamma"); }
        void BatchNorm::set_beta(const Tensor<float, 1>& b) { set_vec(beta_, b, "BatchNorm::set_beta"); }
        void BatchNorm::set_running_mean(const Tensor<float, 1>& m) { set_vec(rmean_, m, "BatchNorm::set_running_mean"); }
        void BatchNorm::set_running_var(const Tensor<float, 1>& v) { set_vec(rvar_, v, "BatchNorm::set_running_var"); }

        // ---------------------------------------------------------------- MeanPool1D
        MeanPool1D::MeanPool1D(const std::string& device) : device_(device)
        {
            require_gpu_device(device_, "MeanPool1D");
        }

        DeviceTensor MeanPool1D::forward(const DeviceTensor& x)
        {
            if (x.rank() != 3) throw std::runtime_error("MeanPool1D::forward: expected [B, S, D]");
            B_ = x.dimension(0);
            S_ = x.dimension(1);
            D_ = x.dimension(2);
            DeviceTensor y = DeviceTensor::empty({B_, D_});
            Device::check(cnhip_meanpool1d_forward_rows(x.data(), y.data(), B_, S_, D_, rows_, Device::stream()),
                          "MeanPool1D::forward");
            return y;
        }

        DeviceTensor MeanPool1D::backward(const DeviceTensor& g)
        {
            if (S_ == 0) throw std::runtime_error("MeanPool1D::backward before forward");
            if (g.rank() != 2 || g.dimension(0) != B_ || g.dimension(1) != D_)
                throw std::runtime_error("MeanPool1D::backward: grad shape " + shape_str(g.dims()));
            DeviceTensor dx = DeviceTensor::empty({B_, S_, D_});
            Device::check(cnhip_meanpool1d_backward_rows(g.data(), dx.data(), B_, S_, D_, rows_, Device::stream()),
                          "MeanPool1D::backward");
            return dx;
        }

        Tensor<float, 2> MeanPool1D::forward(const Tensor<float, 3>& x)
        {
            require_ref_rows(rows_, "MeanPool1D::forward");
            return forward(DeviceTensor::from_host(x)).to_host<float, 2>();
        }
        Tensor<float, 3> MeanPool1D::backward(const Tensor<float, 2>& g)
        {
            require_ref_rows(rows_, "MeanPool1D::backward");
            return backward(DeviceTensor::from_host(g)).to_host<float, 3>();
        }

        void MeanPool1D::set_row_order(int rows) { rows_ = check_rows(rows, "MeanPool1D::set_row_order"); }

        // ---------------------------------------------------------------- Residual
        Residual::Residual(std::vector<std::shared_ptr<Layer>> block, int in_features, int out_features,
                           const std::string& device)
            : block_(std::move(block)), in_features_(in_features), out_features_(out_features), device_(device)
        {
            if (block_.empty()) throw std::invalid_argument("Residual: block must contain at least one layer");
            require_gpu_device(device_, "Residual");
            if (in_features_ != out_features_)  // residual.cpp:31-36
                projection_ = std::make_shared<Linear>(in_features_, out_features_, "ResProj", true, false, device_);
        }

        namespace
        {
            DeviceTensor add(const DeviceTensor& a, const DeviceTensor& b, const char* who)
            {
                if (a.size() != b.size())
                    throw std::runtime_error(std::string(who) + ": shapes " + shape_str(a.dims()) + " and " +
                                             shape_str(b.dims()) + " differ");
                DeviceTensor y = DeviceTensor::empty(a.dims());
                Device::check(cnhip_add(a.data(), b.data(), y.data(), a.size(), Device::stream()), who);
                return y;
            }
        } // namespace

        DeviceTensor Residual::forward(const DeviceTensor& x)
        {
            DeviceTensor out = x;
            for (auto& l : block_)  // only Linear layers run (residual.cpp:48-57)
                if (auto* lin = dynamic_cast<Linear*>(l.get())) out = lin->forward(out);
            DeviceTensor shortcut = projection_ ? projection_->forward(x) : x;
            return add(out, shortcut, "Residual::forward");
        }

        DeviceTensor Residual::backward(const DeviceTensor& g)
        {
            DeviceTensor gb = g;
            for (auto it = block_.rbegin(); it != block_.rend(); ++it)
                if (auto* lin = dynamic_cast<Linear*>(it->get())) gb = lin->backward(gb);
            DeviceTensor gs = projection_ ? projection_->backward(g) : g;
            return add(gb, gs, "Residual::backward");
        }

        Tensor<float, 2> Residual::forward(const Tensor<float, 2>& x)
        {
            return forward(DeviceTensor::from_host(x)).to_host<float, 2>();
        }
        Tensor<float, 2> Residual::backward(const Tensor<float, 2>& g)
        {
            return backward(DeviceTensor::from_host(g)).to_host<float, 2>();
        }

        void Residual::step(Optimizers::Optimizer& optimizer, float learning_rate)
        {
            for (auto& l : block_)
                if (l->is_trainable()) l->step(optimizer, learning_rate);
            if (projection_) projection_->step(optimizer, learning_rate);
        }

        void Residual::reset_grads()
        {
            for (auto& l : block_)
                if (auto* lin = dynamic_cast<Linear*>(l.get())) lin->reset_grads();
            if (projection_) projection_->reset_grads();
        }
    } // namespace Layers

    namespace Activations
    {
        GELU::GELU(const std::string& device) { Layers::require_gpu_device(device, "GELU"); }

        DeviceTensor GELU::forward(const DeviceTensor& x)
        {
            if (!x.defined() || x.size() == 0) throw std::runtime_error("GELU: empty input");
            DeviceTensor y = DeviceTensor::empty(x.dims());
            Device::check(cnhip_gelu_forward(x.data(), y.data(), x.size(), Device::stream()), "GELU");
            in_cache_ = x;
            return y;
        }

        DeviceTensor GELU::backward(const DeviceTensor& g)
        {
            if (!in_cache_.defined() || in_cache_.size() != g.size())
                throw std::runtime_error("GELU: backward before forward or shape mismatch");
            DeviceTensor dx = DeviceTensor::empty(g.dims());
            Device::check(cnhip_gelu_backward(in_cache_.data(), g.data(), dx.data(), g.size(), Device::stream()),
                          "GELU");
            return dx;
        }
    } // namespace Activations
} // namespace CppNet
