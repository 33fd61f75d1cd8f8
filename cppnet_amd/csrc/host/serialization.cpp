// Model files and .npy I/O (ref: src/CppNet/utils/serialization.cpp:26-256,
// src/CppNet/utils/tensor_io.cpp:29-170).  Host-side file formats: the
// device tensors are copied to the host once per tensor on save and uploaded
// once per tensor on load.
#include <cstdint>
#include <cstring>
#include <fstream>
#include <functional>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "CppNet/layers/attention.hpp"
#include "CppNet/layers/batch_norm.hpp"
#include "CppNet/layers/conv2d.hpp"
#include "CppNet/layers/dropout.hpp"
#include "CppNet/layers/embedding.hpp"
#include "CppNet/layers/linear.hpp"
#include "CppNet/layers/lstm.hpp"
#include "CppNet/layers/residual.hpp"
#include "CppNet/models/models.hpp"
#include "CppNet/optimizers/optimizer.hpp"
#include "CppNet/utils/serialization.hpp"
#include "CppNet/utils/tensor_io.hpp"

namespace CppNet
{
    namespace Utils
    {
        namespace
        {
            constexpr int32_t kModelMagic = 0x434E4554;  // "CNET" (serialization.cpp:148)
            constexpr int32_t kExtMagic = 0x434E5831;    // "CNX1"
            constexpr int32_t kRngMagic = 0x434E5253;    // "CNRS": Dropout generator positions

            // ------------------------------------------------------------ records
            void put_i32(std::ostream& os, int32_t v) { os.write(reinterpret_cast<const char*>(&v), 4); }

            int32_t get_i32(std::istream& is, const char* what)
            {
                int32_t v = 0;
                if (!is.read(reinterpret_cast<char*>(&v), 4))
                    throw std::runtime_error(std::string("Truncated model file (reading ") + what + ")");
                return v;
            }

            void put_u64(std::ostream& os, uint64_t v) { os.write(reinterpret_cast<const char*>(&v), 8); }

            uint64_t get_u64(std::istream& is, const char* what)
            {
                uint64_t v = 0;
                if (!is.read(reinterpret_cast<char*>(&v), 8))
                    throw std::runtime_error(std::string("Truncated model file (reading ") + what + ")");
                return v;
            }

            int32_t dim32(int64_t d)
            {
                if (d < 0 || d > INT32_MAX) throw std::runtime_error("Tensor dimension does not fit a model file");
                return static_cast<int32_t>(d);
            }

            void put_record(std::ostream& os, const std::vector<int64_t>& dims, const float* data)
            {
                put_i32(os, static_cast<int32_t>(dims.size()));
                int64_t n = 1;
                for (int64_t d : dims)
                {
                    put_i32(os, dim32(d));
                    n *= d;
                }
                os.write(reinterpret_cast<const char*>(data), static_cast<std::streamsize>(n * 4));
            }

            void put_device_record(std::ostream& os, const DeviceTensor& t)
            {
                std::vector<float> h(static_cast<size_t>(t.size()));
                if (!h.empty()) t.copy_to_host(h.data());
                put_record(os, t.dims(), h.data());
            }

            // one record; `want_rank` > 0 enforces the rank with the reference's message
            std::vector<float> get_record(std::istream& is, std::vector<int64_t>& dims, int want_rank)
            {
                const int32_t nd = get_i32(is, "ndims");
                if (want_rank > 0 && nd != want_rank)
                    throw std::runtime_error("Expected " + std::to_string(want_rank) + "D tensor in model file");
                if (nd < 0 || nd > 8) throw std::runtime_error("Corrupt tensor record in model file");
                dims.assign(static_cast<size_t>(nd), 0);
                int64_t n = 1;
                for (int32_t i = 0; i < nd; ++i)
                {
                    const int32_t d = get_i32(is, "dims");
                    if (d < 0) throw std::runtime_error("Corrupt tensor record in model file");
                    dims[static_cast<size_t>(i)] = d;
                    n *= d;
                }
                std::vector<float> v(static_cast<size_t>(n));
                if (n && !is.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(n * 4)))
                    throw std::runtime_error("Truncated model file (reading tensor data)");
                return v;
            }

            Tensor<float, 2> get_2d(std::istream& is)
            {
                std::vector<int64_t> d;
                auto v = get_record(is, d, 2);
                Tensor<float, 2> t(d[0], d[1]);
                std::memcpy(t.data(), v.data(), v.size() * 4);
                return t;
            }

            Tensor<float, 1> get_1d(std::istream& is)
            {
                std::vector<int64_t> d;
                auto v = get_record(is, d, 1);
                Tensor<float, 1> t(d[0]);
                std::memcpy(t.data(), v.data(), v.size() * 4);
                return t;
            }

            template <int R>
            void put_host(std::ostream& os, const Tensor<float, R>& t)
            {
                std::vector<int64_t> dims(t.dimensions().begin(), t.dimensions().end());
                put_record(os, dims, t.data());
            }

            // ------------------------------------------------------------ parameters
            // The device tensors a trainable layer's step() updates, in that order.
            void layer_params(Layers::Layer* l, std::vector<DeviceTensor*>& out)
            {
                if (auto* p = dynamic_cast<Layers::Linear*>(l))
                {
                    out.push_back(&p->weights());
                    if (p->has_bias()) out.push_back(&p->biases());
                }
                else if (auto* p = dynamic_cast<Layers::Conv2D*>(l))
                {
                    out.push_back(&p->weights());
                    if (p->has_bias()) out.push_back(&p->biases());
                }
                else if (auto* p = dynamic_cast<Layers::RecurrentBase*>(l))
                {
                    out.push_back(&p->W_ih());
                    out.push_back(&p->W_hh());
                    out.push_back(&p->bias());
                }
                else if (auto* p = dynamic_cast<Layers::MultiHeadAttention*>(l))
                {
                    for (int i = 0; i < 4; ++i) out.push_back(&p->weight(i));
                }
                else if (auto* p = dynamic_cast<Layers::BatchNorm*>(l))
                {
                    out.push_back(&p->gamma());
                    out.push_back(&p->beta());
                }
                else if (auto* p = dynamic_cast<Layers::Embedding*>(l))
                {
                    out.push_back(&p->weights());
                }
                else if (auto* p = dynamic_cast<Layers::Residual*>(l))
                {
                    for (std::size_t i = 0; i < p->num_block_layers(); ++i)
                        if (p->block_layer(i)->is_trainable()) layer_params(p->block_layer(i), out);
                    if (p->has_projection()) layer_params(p->projection(), out);
                }
                else
                    throw std::runtime_error("save_checkpoint: no parameter layout known for a trainable layer type");
            }

            // the model's Dropout layers, in order
            std::vector<Layers::Dropout*> dropouts(const std::vector<Layers::Layer*>& layers)
            {
                std::vector<Layers::Dropout*> out;
                for (Layers::Layer* l : layers)
                    if (auto* d = dynamic_cast<Layers::Dropout*>(l)) out.push_back(d);
                return out;
            }

            std::vector<DeviceTensor*> all_params(const std::vector<Layers::Layer*>& layers)
            {
                std::vector<DeviceTensor*> out;
                for (Layers::Layer* l : layers)
                    if (l->is_trainable()) layer_params(l, out);
                return out;
            }

            std::vector<Layers::Layer*> model_layers(const Models::SequentialModel& model)
            {
                std::vector<Layers::Layer*> v;
                for (std::size_t i = 0; i < model.num_layers(); ++i) v.push_back(model.get_layer(i).get());
                return v;
            }

            // ------------------------------------------------------------ CNET section
            // serialization.cpp:143-193
            void write_cnet(std::ostream& os, const std::vector<Layers::Layer*>& layers)
            {
                put_i32(os, kModelMagic);
                put_i32(os, static_cast<int32_t>(layers.size()));
                for (Layers::Layer* l : layers)
                {
                    if (!l->is_trainable()) continue;
                    if (auto* lin = dynamic_cast<Layers::Linear*>(l))
                    {
                        put_i32(os, 1);
                        put_host(os, lin->get_weights());
                        if (lin->has_bias()) put_host(os, lin->get_biases());
                    }
                    else if (auto* bn = dynamic_cast<Layers::BatchNorm*>(l))
                    {
                        put_i32(os, 2);
                        put_host(os, bn->get_gamma());
                        put_host(os, bn->get_beta());
                        put_host(os, bn->get_running_mean());
                        put_host(os, bn->get_running_var());
                    }
                    else if (auto* emb = dynamic_cast<Layers::Embedding*>(l))
                    {
                        put_i32(os, 3);
                        put_host(os, emb->get_weight());
                    }
                    else
                        put_i32(os, 0);
                }
            }

            // A parsed, checked piece of a model file that writes itself into
            // the model when called.  Loading parses and checks the whole file
            // first and applies the pieces only then, so a file that is
            // refused leaves every parameter and optimizer state unchanged.
            using Apply = std::function<void()>;

            void check_dims(const std::vector<int64_t>& got, const std::vector<int64_t>& want, std::size_t idx,
                            const char* what)
            {
                if (got != want)
                    throw std::runtime_error("Shape mismatch at layer index " + std::to_string(idx) + " (" + what +
                                             "): " + shape_str(got) + " in the file, " + shape_str(want) +
                                             " in the model");
            }
            template <int R>
            std::vector<int64_t> dims_of(const Tensor<float, R>& t)
            {
                return std::vector<int64_t>(t.dimensions().begin(), t.dimensions().end());
            }

            // serialization.cpp:195-256: records are matched to the trainable
            // layers in order; what follows the last one is left unread
            std::vector<Apply> read_cnet(std::istream& is, const std::vector<Layers::Layer*>& layers)
            {
                if (get_i32(is, "magic") != kModelMagic) throw std::runtime_error("Invalid model file (bad magic number)");
                const int32_t nlayers = get_i32(is, "layer count");
                std::vector<Apply> out;
                std::size_t idx = 0;
                for (int32_t i = 0; i < nlayers; ++i)
                {
                    while (idx < layers.size() && !layers[idx]->is_trainable()) ++idx;
                    if (idx >= layers.size()) break;
                    Layers::Layer* l = layers[idx];
                    const int32_t type = get_i32(is, "type id");
                    const std::string mismatch = "Layer type mismatch at index " + std::to_string(idx);
                    if (type == 1)
                    {
                        auto* lin = dynamic_cast<Layers::Linear*>(l);
                        if (!lin) throw std::runtime_error(mismatch);
                        Tensor<float, 2> W = get_2d(is);
                        check_dims(dims_of(W), lin->weights().dims(), idx, "Linear weights");
                        Tensor<float, 1> b;
                        if (lin->has_bias())
                        {
                            b = get_1d(is);
                            check_dims(dims_of(b), {lin->get_output_size()}, idx, "Linear biases");
                        }
                        out.push_back([lin, W, b] {
                            lin->set_weights(W);
                            if (lin->has_bias()) lin->set_biases(b);
                        });
                    }
                    else if (type == 2)
                    {
                        auto* bn = dynamic_cast<Layers::BatchNorm*>(l);
                        if (!bn) throw std::runtime_error(mismatch);
                        std::vector<Tensor<float, 1>> v;
                        for (const char* what : {"gamma", "beta", "running mean", "running variance"})
                        {
                            v.push_back(get_1d(is));
                            check_dims(dims_of(v.back()), {bn->get_num_features()}, idx, what);
                        }
                        out.push_back([bn, v] {
                            bn->set_gamma(v[0]);
                            bn->set_beta(v[1]);
                            bn->set_running_mean(v[2]);
                            bn->set_running_var(v[3]);
                        });
                    }
                    else if (type == 3)
                    {
                        auto* emb = dynamic_cast<Layers::Embedding*>(l);
                        if (!emb) throw std::runtime_error(mismatch);
                        Tensor<float, 2> W = get_2d(is);
                        check_dims(dims_of(W), {emb->get_vocab_size(), emb->get_embed_dim()}, idx, "Embedding weight");
                        out.push_back([emb, W] { emb->set_weight(W); });
                    }
                    ++idx;  // type 0 (and unknown ids, as the reference) carry nothing
                }
                return out;
            }

            // ------------------------------------------------------------ extension
            void write_ext(std::ostream& os, const std::vector<Layers::Layer*>& layers,
                           const Optimizers::Optimizer* opt)
            {
                const auto params = all_params(layers);
                put_i32(os, kExtMagic);
                put_i32(os, static_cast<int32_t>(params.size()));
                for (DeviceTensor* p : params) put_device_record(os, *p);
                const int kind = opt ? opt->kind_code() : -1;
                const int S = kind >= 0 ? opt->state_tensors() : 0;
                put_i32(os, kind);
                put_i32(os, S);
                if (kind >= 0)
                {
                    std::vector<std::vector<float>> st;
                    for (DeviceTensor* p : params)
                    {
                        int t = 0;
                        const bool present = opt->get_state(p->data(), p->size(), st, t);
                        put_i32(os, present ? 1 : 0);
                        put_i32(os, t);
                        for (int k = 0; k < S; ++k)
                        {
                            if (present)
                                put_record(os, {p->size()}, st[static_cast<size_t>(k)].data());
                            else
                                put_record(os, {0}, nullptr);
                        }
                    }
                }
                // the mask generators' positions, so a resumed run draws the
                // masks the uninterrupted run would have
                const auto drops = dropouts(layers);
                put_i32(os, kRngMagic);
                put_i32(os, static_cast<int32_t>(drops.size()));
                for (Layers::Dropout* d : drops)
                {
                    put_u64(os, d->rng_seed());
                    put_u64(os, d->rng_offset());
                }
            }

            Apply read_ext(std::istream& is, const std::vector<Layers::Layer*>& layers, Optimizers::Optimizer* opt)
            {
                if (get_i32(is, "extension magic") != kExtMagic)
                    throw std::runtime_error("load_checkpoint: no checkpoint extension after the model records");
                const auto params = all_params(layers);
                const int32_t P = get_i32(is, "parameter count");
                if (P != static_cast<int32_t>(params.size()))
                    throw std::runtime_error("load_checkpoint: the file holds " + std::to_string(P) +
                                             " parameters, the model " + std::to_string(params.size()));
                // read everything before touching the model, so a bad file changes nothing
                std::vector<std::vector<float>> values(params.size());
                for (std::size_t i = 0; i < params.size(); ++i)
                {
                    std::vector<int64_t> dims;
                    values[i] = get_record(is, dims, 0);
                    if (dims != params[i]->dims())
                        throw std::runtime_error("load_checkpoint: parameter " + std::to_string(i) + " has shape " +
                                                 shape_str(dims) + " in the file, " + shape_str(params[i]->dims()) +
                                                 " in the model");
                }
                const int32_t kind = get_i32(is, "optimizer kind");
                const int32_t S = get_i32(is, "optimizer state count");
                struct St
                {
                    bool present;
                    int t;
                    std::vector<std::vector<float>> tensors;
                };
                std::vector<St> states;
                if (kind >= 0)
                {
                    if (S < 0 || S > 8) throw std::runtime_error("load_checkpoint: corrupt optimizer section");
                    for (std::size_t i = 0; i < params.size(); ++i)
                    {
                        St s;
                        s.present = get_i32(is, "state flag") != 0;
                        s.t = get_i32(is, "step count");
                        for (int32_t k = 0; k < S; ++k)
                        {
                            std::vector<int64_t> dims;
                            s.tensors.push_back(get_record(is, dims, 1));
                            if (s.present && dims[0] != params[i]->size())
                                throw std::runtime_error("load_checkpoint: optimizer state size mismatch");
                        }
                        states.push_back(std::move(s));
                    }
                }
                if (opt && kind >= 0 && (kind != opt->kind_code() || S != opt->state_tensors()))
                    throw std::runtime_error("load_checkpoint: the file's optimizer state is of kind " +
                                             std::to_string(kind) + ", the optimizer's kind is " +
                                             std::to_string(opt->kind_code()));
                // Dropout generator positions (absent from files written before
                // this section existed: those leave the generators as they are)
                const auto drops = dropouts(layers);
                std::vector<std::pair<uint64_t, uint64_t>> rng;
                int32_t tag = 0;
                is.read(reinterpret_cast<char*>(&tag), 4);
                if (is.gcount() != 0 && is.gcount() != 4)
                    throw std::runtime_error("Truncated model file: the Dropout section's tag is cut short");
                if (is.gcount() == 4)
                {
                    if (tag != kRngMagic) throw std::runtime_error("load_checkpoint: corrupt extension after the optimizer state");
                    const int32_t n = get_i32(is, "dropout count");
                    if (n != static_cast<int32_t>(drops.size()))
                        throw std::runtime_error("load_checkpoint: the file holds " + std::to_string(n) +
                                                 " Dropout generators, the model has " + std::to_string(drops.size()) +
                                                 " Dropout layers");
                    for (int32_t i = 0; i < n; ++i)
                    {
                        const uint64_t seed = get_u64(is, "dropout seed");
                        rng.emplace_back(seed, get_u64(is, "dropout offset"));
                    }
                }
                return [params, values = std::move(values), opt, kind, states = std::move(states), drops,
                        rng = std::move(rng)] {
                    for (std::size_t i = 0; i < params.size(); ++i)
                        if (!values[i].empty()) params[i]->copy_from_host(values[i].data());
                    if (opt && kind >= 0)
                        for (std::size_t i = 0; i < params.size(); ++i)
                            if (states[i].present)
                                opt->set_state(params[i]->data(), params[i]->size(), states[i].tensors, states[i].t);
                    for (std::size_t i = 0; i < rng.size(); ++i) drops[i]->set_rng_state(rng[i].first, rng[i].second);
                };
            }

            // ------------------------------------------------------------ .npy
            // tensor_io.cpp:29-58, with the order flag telling the truth
            void write_npy_header(std::ostream& os, const std::vector<int64_t>& dims)
            {
                std::ostringstream d;
                d << "{'descr': '<f4', 'fortran_order': True, 'shape': (";
                for (std::size_t i = 0; i < dims.size(); ++i)
                {
                    d << dims[i];
                    if (i + 1 < dims.size()) d << ", ";
                }
                if (dims.size() == 1) d << ",";
                d << "), }\n";
                std::string s = d.str();
                const std::size_t pad = (64 - (10 + s.size()) % 64) % 64;
                s.insert(s.size() - 1, pad, ' ');
                if (s.size() > 65535) throw std::runtime_error("save_npy: header too long");
                const uint16_t len = static_cast<uint16_t>(s.size());
                os.write("\x93NUMPY", 6);
                const char ver[2] = {1, 0};
                os.write(ver, 2);
                os.write(reinterpret_cast<const char*>(&len), 2);
                os.write(s.data(), static_cast<std::streamsize>(s.size()));
            }

            // tensor_io.cpp:60-100; versions 1.0 to 3.0 (4-byte length from 2.0)
            std::vector<int64_t> read_npy_header(std::istream& is, bool& fortran)
            {
                char magic[6];
                if (!is.read(magic, 6) || std::memcmp(magic, "\x93NUMPY", 6) != 0)
                    throw std::runtime_error("Not a valid .npy file (bad magic)");
                unsigned char ver[2];
                is.read(reinterpret_cast<char*>(ver), 2);
                uint32_t len = 0;
                if (ver[0] == 1)
                {
                    uint16_t l16 = 0;
                    is.read(reinterpret_cast<char*>(&l16), 2);
                    len = l16;
                }
                else if (ver[0] == 2 || ver[0] == 3)
                    is.read(reinterpret_cast<char*>(&len), 4);
                else
                    throw std::runtime_error("Unsupported .npy version " + std::to_string(ver[0]));
                if (!is || len > (1u << 24)) throw std::runtime_error("Malformed .npy header");
                std::string h(len, ' ');
                if (!is.read(&h[0], len)) throw std::runtime_error("Truncated .npy header");
                if (h.find("<f4") == std::string::npos)
                    throw std::runtime_error("Only float32 (<f4) .npy files are supported");
                const auto fo = h.find("'fortran_order':");
                if (fo == std::string::npos) throw std::runtime_error("Malformed .npy header: missing fortran_order");
                fortran = h.compare(h.find_first_not_of(' ', fo + 16), 4, "True") == 0;
                auto a = h.find("'shape': (");
                if (a == std::string::npos) throw std::runtime_error("Malformed .npy header: missing shape");
                a += 10;
                const auto b = h.find(')', a);
                if (b == std::string::npos) throw std::runtime_error("Malformed .npy header: missing shape");
                std::vector<int64_t> dims;
                std::istringstream ss(h.substr(a, b - a));
                std::string tok;
                while (std::getline(ss, tok, ','))
                {
                    const auto s0 = tok.find_first_not_of(' ');
                    if (s0 == std::string::npos) continue;
                    dims.push_back(std::stoll(tok.substr(s0)));
                }
                return dims;
            }

            template <int R>
            Tensor<float, R> load_npy_r(const std::string& path, bool raw)
            {
                std::vector<int64_t> dims;
                std::vector<float> v = load_npy_raw(path, dims, raw);
                if (static_cast<int>(dims.size()) != R)
                    throw std::runtime_error("Expected " + std::to_string(R) + "D tensor in " + path);
                typename Tensor<float, R>::Dimensions d;
                for (int i = 0; i < R; ++i) d[static_cast<size_t>(i)] = dims[static_cast<size_t>(i)];
                Tensor<float, R> t(d);
                if (!v.empty()) std::memcpy(t.data(), v.data(), v.size() * 4);
                return t;
            }

            template <int R>
            void save_npy_r(const std::string& path, const Tensor<float, R>& t)
            {
                std::vector<int64_t> dims(t.dimensions().begin(), t.dimensions().end());
                save_npy_raw(path, t.data(), dims);
            }
        } // namespace

        // ---------------------------------------------------------------- tensors
        void save_tensor(const std::string& path, const Tensor<float, 2>& t)
        {
            std::ofstream os(path, std::ios::binary);
            if (!os) throw std::runtime_error("Cannot open file for writing: " + path);
            put_host(os, t);
        }

        void save_tensor(const std::string& path, const Tensor<float, 1>& t)
        {
            std::ofstream os(path, std::ios::binary);
            if (!os) throw std::runtime_error("Cannot open file for writing: " + path);
            put_host(os, t);
        }

        Tensor<float, 2> load_tensor_2d(const std::string& path)
        {
            std::ifstream is(path, std::ios::binary);
            if (!is) throw std::runtime_error("Cannot open file for reading: " + path);
            const int32_t nd = get_i32(is, "ndims");
            if (nd != 2) throw std::runtime_error("Expected 2D tensor, got " + std::to_string(nd) + "D");
            is.seekg(0);
            return get_2d(is);
        }

        Tensor<float, 1> load_tensor_1d(const std::string& path)
        {
            std::ifstream is(path, std::ios::binary);
            if (!is) throw std::runtime_error("Cannot open file for reading: " + path);
            const int32_t nd = get_i32(is, "ndims");
            if (nd != 1) throw std::runtime_error("Expected 1D tensor, got " + std::to_string(nd) + "D");
            is.seekg(0);
            return get_1d(is);
        }

        // ---------------------------------------------------------------- models
        void save_layers(const std::string& path, const std::vector<Layers::Layer*>& layers,
                         const Optimizers::Optimizer* optimizer, bool extension)
        {
            // serialize into memory first: a failure leaves no partial file behind
            std::ostringstream buf(std::ios::binary);
            write_cnet(buf, layers);
            if (extension) write_ext(buf, layers, optimizer);
            std::ofstream os(path, std::ios::binary);
            if (!os) throw std::runtime_error("Cannot open file for writing: " + path);
            const std::string s = buf.str();
            if (!os.write(s.data(), static_cast<std::streamsize>(s.size())))
                throw std::runtime_error("Write failed: " + path);
        }

        void load_layers(const std::string& path, const std::vector<Layers::Layer*>& layers,
                         Optimizers::Optimizer* optimizer, bool extension)
        {
            std::ifstream is(path, std::ios::binary);
            if (!is) throw std::runtime_error("Cannot open file for reading: " + path);
            const std::vector<Apply> records = read_cnet(is, layers);
            Apply ext;
            if (extension) ext = read_ext(is, layers, optimizer);
            for (const Apply& a : records) a();
            if (ext) ext();
        }

        void save_model(const std::string& path, const Models::SequentialModel& model)
        {
            save_layers(path, model_layers(model), nullptr, false);
        }

        void load_model(const std::string& path, Models::SequentialModel& model)
        {
            load_layers(path, model_layers(model), nullptr, false);
        }

        void save_checkpoint(const std::string& path, const Models::SequentialModel& model,
                             const Optimizers::Optimizer* optimizer)
        {
            save_layers(path, model_layers(model), optimizer, true);
        }

        void load_checkpoint(const std::string& path, Models::SequentialModel& model, Optimizers::Optimizer* optimizer)
        {
            load_layers(path, model_layers(model), optimizer, true);
        }

        // ---------------------------------------------------------------- .npy
        void save_npy_raw(const std::string& path, const float* colmajor, const std::vector<int64_t>& dims)
        {
            if (dims.empty()) throw std::invalid_argument("save_npy: rank must be at least 1");
            int64_t n = 1;
            for (int64_t d : dims)
            {
                if (d < 0) throw std::invalid_argument("save_npy: negative dimension");
                n *= d;
            }
            std::ofstream os(path, std::ios::binary);
            if (!os) throw std::runtime_error("Cannot open " + path + " for writing");
            write_npy_header(os, dims);
            os.write(reinterpret_cast<const char*>(colmajor), static_cast<std::streamsize>(n * 4));
            if (!os) throw std::runtime_error("Write failed: " + path);
        }

        std::vector<float> load_npy_raw(const std::string& path, std::vector<int64_t>& dims, bool raw_colmajor)
        {
            std::ifstream is(path, std::ios::binary);
            if (!is) throw std::runtime_error("Cannot open " + path + " for reading");
            bool fortran = false;
            dims = read_npy_header(is, fortran);
            if (dims.empty()) throw std::runtime_error("Scalar .npy files are not supported: " + path);
            int64_t n = 1;
            for (int64_t d : dims)
            {
                if (d < 0) throw std::runtime_error("Malformed .npy shape in " + path);
                n *= d;
            }
            std::vector<float> v(static_cast<size_t>(n));
            if (n && !is.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(n * 4)))
                throw std::runtime_error("Truncated .npy data in " + path);
            if (fortran || raw_colmajor || dims.size() == 1) return v;
            // C order -> ColMajor: element (i0, ..., ik) sits at the row-major
            // offset in v and goes to the column-major offset
            const std::size_t R = dims.size();
            std::vector<int64_t> cstride(R), fstride(R);
            cstride[R - 1] = 1;
            for (std::size_t k = R - 1; k-- > 0;) cstride[k] = cstride[k + 1] * dims[k + 1];
            fstride[0] = 1;
            for (std::size_t k = 1; k < R; ++k) fstride[k] = fstride[k - 1] * dims[k - 1];
            std::vector<float> out(static_cast<size_t>(n));
            std::vector<int64_t> idx(R, 0);
            for (int64_t c = 0; c < n; ++c)
            {
                int64_t f = 0;
                for (std::size_t k = 0; k < R; ++k) f += idx[k] * fstride[k];
                out[static_cast<size_t>(f)] = v[static_cast<size_t>(c)];
                for (std::size_t k = R; k-- > 0;)  // advance the row-major index
                {
                    if (++idx[k] < dims[k]) break;
                    idx[k] = 0;
                }
            }
            return out;
        }

        void save_npy(const std::string& path, const Tensor<float, 1>& t) { save_npy_r(path, t); }
        void save_npy(const std::string& path, const Tensor<float, 2>& t) { save_npy_r(path, t); }
        void save_npy(const std::string& path, const Tensor<float, 3>& t) { save_npy_r(path, t); }
        void save_npy(const std::string& path, const Tensor<float, 4>& t) { save_npy_r(path, t); }

        void save_npy(const std::string& path, const DeviceTensor& t)
        {
            std::vector<float> h(static_cast<size_t>(t.size()));
            if (!h.empty()) t.copy_to_host(h.data());
            save_npy_raw(path, h.data(), t.dims());
        }

        Tensor<float, 1> load_npy_1d(const std::string& path, bool raw) { return load_npy_r<1>(path, raw); }
        Tensor<float, 2> load_npy_2d(const std::string& path, bool raw) { return load_npy_r<2>(path, raw); }
        Tensor<float, 3> load_npy_3d(const std::string& path, bool raw) { return load_npy_r<3>(path, raw); }
        Tensor<float, 4> load_npy_4d(const std::string& path, bool raw) { return load_npy_r<4>(path, raw); }
    } // namespace Utils
} // namespace CppNet
