// Training harness C ABI (include/cppnet_train.h): builds models from the
// CppNet-compatible classes and runs the reference harness's train step.
#include "cppnet_train.h"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <exception>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "CppNet/CppNet.hpp"
#include "CppNet/utils/serialization.hpp"
#include "CppNet/utils/tensor_io.hpp"
#include "CppNet/utils/dataloader.hpp"

using namespace CppNet;

namespace
{
    /**
     * Config-5 encoder block, composed by the harness as the reference's
     * harness composes its layers (no encoder class exists in the reference):
     *   r = MHA(x, x, x) + x;  h = BatchNorm(r as [B*S, D]);
     *   y = Linear2(GELU(Linear1(h))) + h
     */
    struct EncoderBlock
    {
        std::shared_ptr<Layers::MultiHeadAttention> mha;
        std::shared_ptr<Layers::BatchNorm> bn;
        std::shared_ptr<Layers::Linear> ff1, ff2;
        std::shared_ptr<Activations::GELU> gelu;
        std::vector<int64_t> dims;

        // The four skip sums run in the epilogues of the GEMMs that produce
        // their other operand (MHA's output projection and input gradient,
        // the second FFN Linear's output, the first FFN Linear's input
        // gradient): the same additions as separate adds, one pass fewer each.
        DeviceTensor forward(const DeviceTensor& x)
        {
            dims = x.dims();
            const int64_t BS = dims[0] * dims[1], D = dims[2];
            DeviceTensor r = mha->forward_residual(x, x, x, x);
            DeviceTensor h = bn->forward(r.reshape({BS, D}));
            // GELU runs as its own pass in the forward (fused into the first
            // FFN GEMM's epilogue it measured slower: the erfc work serialises
            // after the MFMA loop); its derivative is fused into the second
            // FFN GEMM's input gradient
            DeviceTensor f = ff2->forward_residual(gelu->forward(ff1->forward(h)), h);
            return f.reshape(dims);
        }

        DeviceTensor backward(const DeviceTensor& g)
        {
            const int64_t BS = dims[0] * dims[1], D = dims[2];
            DeviceTensor g2 = g.reshape({BS, D});
            DeviceTensor gz = ff2->backward_act(g2, CNHIP_ACT_GELU, gelu->input_cache());
            DeviceTensor gh = ff1->backward_act(gz, CNHIP_ACT_RESIDUAL, g2);
            DeviceTensor gr = bn->backward(gh).reshape(dims);
            return mha->backward_residual(gr, gr);
        }

        void step(Optimizers::Optimizer& opt, float lr)
        {
            mha->step(opt, lr);
            bn->step(opt, lr);
            ff1->step(opt, lr);
            ff2->step(opt, lr);
        }

        void zero_grad()
        {
            mha->reset_grads();
            bn->reset_grads();
            ff1->reset_grads();
            ff2->reset_grads();
        }
    };

    /// Embedding -> blocks -> MeanPool1D -> Linear (logits).
    struct EncoderNet
    {
        std::shared_ptr<Layers::Embedding> emb;
        std::vector<EncoderBlock> blocks;
        std::shared_ptr<Layers::MeanPool1D> pool;
        std::shared_ptr<Layers::Linear> fc;

        DeviceTensor forward(const DeviceTensor& ids)
        {
            DeviceTensor x = emb->forward(ids, /*ids_checked=*/true);  // checked at upload
            for (auto& b : blocks) x = b.forward(x);
            return fc->forward(pool->forward(x));
        }

        void backward(const DeviceTensor& g)
        {
            DeviceTensor x = pool->backward(fc->backward(g));
            for (auto it = blocks.rbegin(); it != blocks.rend(); ++it) x = it->backward(x);
            emb->backward(x, false);  // the ids take no gradient
        }

        void update(Optimizers::Optimizer& opt, float lr)
        {
            opt.begin_group();
            try
            {
                emb->step(opt, lr);
                for (auto& b : blocks) b.step(opt, lr);
                fc->step(opt, lr);
            }
            catch (...)
            {
                opt.end_group();
                throw;
            }
            opt.end_group();
        }

        void zero_grad()
        {
            emb->reset_grads();
            for (auto& b : blocks) b.zero_grad();
            fc->reset_grads();
        }
    };
} // namespace

struct cnt_session
{
    cnhip_stream_t stream = nullptr;
    Models::SequentialModel model;
    std::unique_ptr<EncoderNet> encoder;  // set for transformer sessions (X holds int32 ids)
    std::vector<std::shared_ptr<Layers::Layer>> keep;  // owns the layers
    std::unique_ptr<Losses::Loss> loss;
    std::unique_ptr<Optimizers::Optimizer> opt;  // Adam unless cnt_set_optimizer replaced it
    bool updated = false;                        // an optimizer update has run
    bool fused_steps = true;                     // cnt_set_fused_step
    bool fused_taken = false;                    // a fused step has run (cnt_capture_step)
    float lr = 1e-3f;
    DeviceTensor X, Y;
    Losses::DeviceScalar last_loss;

    // Captured forward + backward (cnt_capture_step): replayed by cnt_step,
    // followed by the eager Adam update.  The graph writes its loss into
    // graph_loss; its memory is the allocator pool graph_pool.
    bool warm = false;  // one eager forward + backward has run at the batch shapes
    cnhip_graph_t graph = nullptr;
    uint64_t graph_pool = 0;
    Losses::DeviceScalar graph_loss;
    // each layer's grads_pending_zero() as the captured backward leaves it
    std::vector<std::pair<Layers::Layer*, bool>> graph_flags;

    std::vector<Layers::Layer*> all_layers()
    {
        std::vector<Layers::Layer*> out;
        for (std::size_t i = 0; i < model.num_layers(); ++i) out.push_back(model.get_layer(i).get());
        if (encoder)
        {
            out.push_back(encoder->emb.get());
            for (auto& b : encoder->blocks)
                for (Layers::Layer* l : {static_cast<Layers::Layer*>(b.mha.get()),
                                         static_cast<Layers::Layer*>(b.bn.get()),
                                         static_cast<Layers::Layer*>(b.ff1.get()),
                                         static_cast<Layers::Layer*>(b.ff2.get())})
                    out.push_back(l);
            out.push_back(encoder->fc.get());
        }
        return out;
    }

    // parameter index -> accessors of the value and of the gradient, called
    // through the layer so lazily-zeroed gradients are materialised first
    struct Param
    {
        std::function<DeviceTensor&()> value, grad;
        // > 0: stored as the transpose of the reference's ColMajor
        // [t_rows, t_cols] (the token-major embedding table)
        int64_t t_rows = 0, t_cols = 0;
    };
    std::vector<Param> params;

    template <class L>
    void add_params(const std::shared_ptr<L>& l)
    {
        add_params(l.get());
    }
    template <class L>
    void add_params(L* p)
    {
        params.push_back({[p]() -> DeviceTensor& { return p->weights(); },
                          [p]() -> DeviceTensor& { return p->grad_weights(); }});
        if (p->has_bias())
            params.push_back({[p]() -> DeviceTensor& { return p->biases(); },
                              [p]() -> DeviceTensor& { return p->grad_biases(); }});
    }
};

namespace
{
    thread_local std::string g_err;

    int fail(int status, const std::string& msg)
    {
        g_err = msg;
        return status;
    }

    template <class F>
    int guarded(const char* who, F&& f)
    {
        try
        {
            f();
            return CNHIP_OK;
        }
        catch (const Device::Error& e)
        {
            return fail(e.status(), std::string(who) + ": " + e.what());
        }
        catch (const std::exception& e)
        {
            return fail(CNHIP_EINVAL, std::string(who) + ": " + e.what());
        }
    }

    // Makes the session's stream the backend stream for the duration of a call.
    struct StreamScope
    {
        cnhip_stream_t saved;
        explicit StreamScope(cnt_session* s) : saved(Device::stream()) { Device::set_stream(s->stream); }
        ~StreamScope() { Device::set_stream(saved); }
    };

    std::shared_ptr<Activations::Activation> make_act(int act)
    {
        switch (act)
        {
            case CNT_ACT_NONE: return nullptr;
            case CNT_ACT_RELU: return std::make_shared<Activations::ReLU>("gpu");
            case CNT_ACT_SIGMOID: return std::make_shared<Activations::Sigmoid>("gpu");
            case CNT_ACT_TANH: return std::make_shared<Activations::Tanh>("gpu");
            case CNT_ACT_LEAKY_RELU: return std::make_shared<Activations::LeakyReLU>(0.01f, "gpu");
            case CNT_ACT_SOFTMAX: return std::make_shared<Activations::Softmax>("gpu");
        }
        throw std::invalid_argument("unknown activation code " + std::to_string(act));
    }

    std::unique_ptr<Losses::Loss> make_loss(int loss)
    {
        switch (loss)
        {
            case CNT_LOSS_BCE: return std::make_unique<Losses::BinaryCrossEntropy>("mean", false, 1.0f, "gpu");
            case CNT_LOSS_SOFTMAX_CE: return std::make_unique<Losses::SoftmaxCrossEntropy>("mean", "gpu");
            case CNT_LOSS_MSE: return std::make_unique<Losses::MSE>("mean", "gpu");
            case CNT_LOSS_CCE:
                return std::make_unique<Losses::CategoricalCrossEntropy>("mean", true, 0.0f, "gpu");
            case CNT_LOSS_MAE: return std::make_unique<Losses::MAE>("mean", "gpu");
            case CNT_LOSS_HUBER: return std::make_unique<Losses::Huber>(1.0f, "mean", "gpu");
        }
        throw std::invalid_argument("unknown loss code " + std::to_string(loss));
    }

    // outputs up to this size take the one-launch Sigmoid + BCE head
    constexpr int64_t kFusedHeadMax = 1 << 16;

    void check_session(cnt_session* s)
    {
        if (!s) throw std::invalid_argument("NULL session");
    }

    cnt_session::Param& param_rec(cnt_session* s, int index)
    {
        check_session(s);
        if (index < 0 || index >= static_cast<int>(s->params.size()))
            throw std::out_of_range("parameter index " + std::to_string(index) + " out of range");
        return s->params[static_cast<size_t>(index)];
    }

    DeviceTensor& param_at(cnt_session* s, int index, bool grad)
    {
        auto& p = param_rec(s, index);
        return grad ? p.grad() : p.value();
    }

    // host copy in the reference's layout
    void param_to_host(cnt_session* s, int index, bool grad, float* host)
    {
        auto& p = param_rec(s, index);
        DeviceTensor& t = grad ? p.grad() : p.value();
        if (p.t_rows == 0)
        {
            t.copy_to_host(host);
            return;
        }
        DeviceTensor tmp = DeviceTensor::empty({p.t_rows, p.t_cols});
        Device::check(cnhip_transpose(t.data(), tmp.data(), p.t_cols, p.t_rows, Device::stream()), "param");
        tmp.copy_to_host(host);
    }

    void param_from_host(cnt_session* s, int index, const float* host)
    {
        auto& p = param_rec(s, index);
        DeviceTensor& t = p.value();
        if (p.t_rows == 0)
        {
            t.copy_from_host(host);
            return;
        }
        DeviceTensor tmp = DeviceTensor::empty({p.t_rows, p.t_cols});
        tmp.copy_from_host(host);
        Device::check(cnhip_transpose(tmp.data(), t.data(), p.t_rows, p.t_cols, Device::stream()), "param");
        Device::synchronize();
    }

    // Destroys the session's captured graph (synchronising its stream) and
    // returns the graph's memory pool to the allocator.
    void release_graph(cnt_session* s)
    {
        if (!s->graph) return;
        cnhip_graph_t g = s->graph;
        s->graph = nullptr;
        s->graph_loss = Losses::DeviceScalar();
        s->graph_flags.clear();
        const int st = cnhip_graph_destroy(g);
        Device::release_pool(s->graph_pool);
        s->graph_pool = 0;
        Device::check(st, "graph");
    }

    std::unique_ptr<cnt_session> new_session(uint64_t seed)
    {
        auto s = std::make_unique<cnt_session>();
        Device::check(cnhip_stream_create(&s->stream), "stream");
        Utils::set_seed(seed);
        return s;
    }
} // namespace

extern "C" {

const char* cnt_last_error(void) { return g_err.c_str(); }

int cnt_mlp_create(cnt_session** out, int n_linear, const int64_t* sizes, int hidden_act, int out_act,
                   int loss, int64_t batch, float lr, float beta1, float beta2, float eps, uint64_t seed)
{
    return cnt_mlp_create_ex(out, n_linear, sizes, hidden_act, out_act, loss, batch, lr, beta1, beta2, eps, seed,
                             0.0f);
}

int cnt_mlp_create_ex(cnt_session** out, int n_linear, const int64_t* sizes, int hidden_act, int out_act,
                      int loss, int64_t batch, float lr, float beta1, float beta2, float eps, uint64_t seed,
                      float dropout)
{
    return guarded("cnt_mlp_create", [&] {
        if (!out) throw std::invalid_argument("NULL out pointer");
        *out = nullptr;
        if (n_linear < 1 || !sizes) throw std::invalid_argument("need at least one Linear layer");
        if (batch <= 0) throw std::invalid_argument("batch must be positive");
        if (!(dropout >= 0.0f && dropout < 1.0f)) throw std::invalid_argument("dropout must be in [0, 1)");
        auto s = new_session(seed);
        StreamScope scope(s.get());
        for (int i = 0; i < n_linear; ++i)
        {
            auto lin = std::make_shared<Layers::Linear>(static_cast<int>(sizes[i]),
                                                        static_cast<int>(sizes[i + 1]),
                                                        "fc" + std::to_string(i + 1), true, true, "gpu",
                                                        "xavier");
            s->model.add_layer(lin);
            s->keep.push_back(lin);
            s->add_params(lin);
            auto act = make_act(i + 1 < n_linear ? hidden_act : out_act);
            if (act) s->model.add_activation(act);
            if (dropout > 0.0f && i + 1 < n_linear)
            {
                auto drop = std::make_shared<Layers::Dropout>(dropout, "gpu");
                s->model.add_layer(drop);
                s->keep.push_back(drop);
            }
        }
        s->loss = make_loss(loss);
        s->opt = std::make_unique<Optimizers::Adam>(beta1, beta2, eps, "gpu");
        s->lr = lr;
        s->X = DeviceTensor::zeros({batch, sizes[0]});
        s->Y = DeviceTensor::zeros({batch, sizes[n_linear]});
        Device::synchronize();
        *out = s.release();
    });
}

int cnt_cnn_create(cnt_session** out, int n_conv, const int64_t* conv_spec, int pool,
                   const int64_t* input_shape, int64_t classes, float lr, float beta1, float beta2,
                   float eps, uint64_t seed)
{
    return guarded("cnt_cnn_create", [&] {
        if (!out) throw std::invalid_argument("NULL out pointer");
        *out = nullptr;
        if (n_conv < 1 || !conv_spec || !input_shape) throw std::invalid_argument("need at least one Conv2D block");
        auto s = new_session(seed);
        StreamScope scope(s.get());
        int64_t C = input_shape[1], H = input_shape[2], W = input_shape[3];
        for (int i = 0; i < n_conv; ++i)
        {
            const int64_t* c = conv_spec + 5 * i;  // in, out, kernel, stride, padding
            if (c[0] != C) throw std::invalid_argument("conv block " + std::to_string(i) + ": in_channels mismatch");
            auto conv = std::make_shared<Layers::Conv2D>(static_cast<int>(c[0]), static_cast<int>(c[1]),
                                                         static_cast<int>(c[2]), static_cast<int>(c[3]),
                                                         static_cast<int>(c[4]), true, "gpu");
            s->model.add_layer(conv);
            s->keep.push_back(conv);
            s->add_params(conv);
            s->model.add_activation(std::make_shared<Activations::ReLU>("gpu"));
            auto mp = std::make_shared<Layers::MaxPool2D>(pool, -1, "gpu");
            s->model.add_layer(mp);
            s->keep.push_back(mp);
            C = c[1];
            H = ((H + 2 * c[4] - c[2]) / c[3] + 1 - pool) / pool + 1;
            W = ((W + 2 * c[4] - c[2]) / c[3] + 1 - pool) / pool + 1;
        }
        auto fl = std::make_shared<Layers::Flatten>();
        s->model.add_layer(fl);
        s->keep.push_back(fl);
        auto fc = std::make_shared<Layers::Linear>(static_cast<int>(C * H * W), static_cast<int>(classes),
                                                   "fc", true, true, "gpu", "xavier");
        s->model.add_layer(fc);
        s->keep.push_back(fc);
        s->add_params(fc);
        s->loss = make_loss(CNT_LOSS_SOFTMAX_CE);
        s->opt = std::make_unique<Optimizers::Adam>(beta1, beta2, eps, "gpu");
        s->lr = lr;
        s->X = DeviceTensor::zeros({input_shape[0], input_shape[1], input_shape[2], input_shape[3]});
        s->Y = DeviceTensor::zeros({input_shape[0], classes});
        Device::synchronize();
        *out = s.release();
    });
}

int cnt_rnn_create(cnt_session** out, int cell, int64_t batch, int64_t seq_len, int64_t input_size,
                   int64_t hidden_size, int64_t out_features, float lr, float beta1, float beta2,
                   float eps, uint64_t seed)
{
    return guarded("cnt_rnn_create", [&] {
        if (!out) throw std::invalid_argument("NULL out pointer");
        *out = nullptr;
        if (batch <= 0 || seq_len <= 0) throw std::invalid_argument("batch and seq_len must be positive");
        auto s = new_session(seed);
        StreamScope scope(s.get());
        std::shared_ptr<Layers::RecurrentBase> rnn;
        if (cell == 0)
        {
            auto l = std::make_shared<Layers::LSTM>(static_cast<int>(input_size), static_cast<int>(hidden_size),
                                                    true, "gpu");
            s->model.add_layer(l);
            rnn = l;
        }
        else if (cell == 1)
        {
            auto g = std::make_shared<Layers::GRU>(static_cast<int>(input_size), static_cast<int>(hidden_size),
                                                   true, "gpu");
            s->model.add_layer(g);
            rnn = g;
        }
        else if (cell == 2)
        {
            auto e = std::make_shared<Layers::RNN>(static_cast<int>(input_size), static_cast<int>(hidden_size),
                                                   true, "gpu");
            s->model.add_layer(e);
            rnn = e;
        }
        else
            throw std::invalid_argument("cell must be 0 (LSTM), 1 (GRU) or 2 (RNN)");
        s->keep.push_back(rnn);
        Layers::RecurrentBase* r = rnn.get();
        s->params.push_back({[r]() -> DeviceTensor& { return r->W_ih(); },
                             [r]() -> DeviceTensor& { return r->grad_W_ih(); }});
        s->params.push_back({[r]() -> DeviceTensor& { return r->W_hh(); },
                             [r]() -> DeviceTensor& { return r->grad_W_hh(); }});
        s->params.push_back({[r]() -> DeviceTensor& { return r->bias(); },
                             [r]() -> DeviceTensor& { return r->grad_bias(); }});
        auto last = std::make_shared<Layers::SequenceLast>();
        s->model.add_layer(last);
        s->keep.push_back(last);
        auto fc = std::make_shared<Layers::Linear>(static_cast<int>(hidden_size), static_cast<int>(out_features),
                                                   "fc", true, true, "gpu", "xavier");
        s->model.add_layer(fc);
        s->keep.push_back(fc);
        s->add_params(fc);
        s->loss = make_loss(CNT_LOSS_MSE);
        s->opt = std::make_unique<Optimizers::Adam>(beta1, beta2, eps, "gpu");
        s->lr = lr;
        s->X = DeviceTensor::zeros({batch, seq_len, input_size});
        s->Y = DeviceTensor::zeros({batch, out_features});
        Device::synchronize();
        *out = s.release();
    });
}

int cnt_resnet_create(cnt_session** out, int64_t in_features, int64_t width, int depth, int64_t last_width,
                      int64_t classes, int64_t batch, float lr, float beta1, float beta2, float eps, uint64_t seed)
{
    return guarded("cnt_resnet_create", [&] {
        if (!out) throw std::invalid_argument("NULL out pointer");
        *out = nullptr;
        if (in_features <= 0 || width <= 0 || depth < 0 || last_width <= 0 || classes <= 0 || batch <= 0)
            throw std::invalid_argument("sizes must be positive and depth >= 0");
        auto s = new_session(seed);
        StreamScope scope(s.get());
        const int W = static_cast<int>(width);
        // residual_benckmark.cpp:108-152: proj (he) -> ReLU -> [Residual -> ReLU] x depth -> head (xavier)
        auto proj = std::make_shared<Layers::Linear>(static_cast<int>(in_features), W, "proj", true, true, "gpu", "he");
        s->model.add_layer(proj);
        s->keep.push_back(proj);
        s->add_params(proj);
        s->model.add_activation(std::make_shared<Activations::ReLU>("gpu"));
        int w = W;
        for (int d = 0; d < depth; ++d)
        {
            const std::string tag = "res" + std::to_string(d);
            const int w_out = d + 1 == depth ? static_cast<int>(last_width) : W;
            auto fc_a = std::make_shared<Layers::Linear>(w, W, tag + "_a", true, true, "gpu", "he");
            auto fc_b = std::make_shared<Layers::Linear>(W, w_out, tag + "_b", true, true, "gpu", "he");
            std::vector<std::shared_ptr<Layers::Layer>> block = {fc_a, fc_b};
            auto res = std::make_shared<Layers::Residual>(block, w, w_out, "gpu");
            s->model.add_layer(res);
            s->keep.push_back(res);
            s->add_params(fc_a);
            s->add_params(fc_b);
            if (res->has_projection()) s->add_params(res->projection());
            s->model.add_activation(std::make_shared<Activations::ReLU>("gpu"));
            w = w_out;
        }
        auto head = std::make_shared<Layers::Linear>(w, static_cast<int>(classes), "head", true, true, "gpu", "xavier");
        s->model.add_layer(head);
        s->keep.push_back(head);
        s->add_params(head);
        s->loss = make_loss(CNT_LOSS_SOFTMAX_CE);
        s->opt = std::make_unique<Optimizers::Adam>(beta1, beta2, eps, "gpu");
        s->lr = lr;
        s->X = DeviceTensor::zeros({batch, in_features});
        s->Y = DeviceTensor::zeros({batch, classes});
        Device::synchronize();
        *out = s.release();
    });
}

int cnt_transformer_create(cnt_session** out, int64_t batch, int64_t seq_len, int64_t vocab,
                           int64_t embed_dim, int64_t heads, int n_blocks, int64_t ffn_dim,
                           int64_t classes, float lr, float beta1, float beta2, float eps, uint64_t seed)
{
    return guarded("cnt_transformer_create", [&] {
        if (!out) throw std::invalid_argument("NULL out pointer");
        *out = nullptr;
        if (batch <= 0 || seq_len <= 0 || n_blocks < 0 || classes <= 0)
            throw std::invalid_argument("batch, seq_len, classes must be positive and n_blocks >= 0");
        auto s = new_session(seed);
        StreamScope scope(s.get());
        auto net = std::make_unique<EncoderNet>();
        const int D = static_cast<int>(embed_dim);
        net->emb = std::make_shared<Layers::Embedding>(static_cast<int>(vocab), D, "gpu");
        // The session owns the whole Embedding -> MeanPool1D chain, so its
        // sequences run by sample (row s + S*b): the attention products then
        // read each sample's rows in place, with no transposes.
        net->emb->set_row_order(CNHIP_ROWS_BY_SAMPLE);
        {
            Layers::Embedding* e = net->emb.get();
            cnt_session::Param p{[e]() -> DeviceTensor& { return e->weights(); },
                                 [e]() -> DeviceTensor& { return e->grad_weights(); }};
            p.t_rows = vocab;
            p.t_cols = embed_dim;
            s->params.push_back(p);
        }
        for (int i = 0; i < n_blocks; ++i)
        {
            EncoderBlock b;
            b.mha = std::make_shared<Layers::MultiHeadAttention>(D, static_cast<int>(heads), "gpu");
            b.mha->set_row_order(CNHIP_ROWS_BY_SAMPLE);
            b.bn = std::make_shared<Layers::BatchNorm>(D, 0.1f, 1e-5f, "gpu");
            b.ff1 = std::make_shared<Layers::Linear>(D, static_cast<int>(ffn_dim), "ffn1_" + std::to_string(i),
                                                     true, true, "gpu", "xavier");
            b.gelu = std::make_shared<Activations::GELU>("gpu");
            b.ff2 = std::make_shared<Layers::Linear>(static_cast<int>(ffn_dim), D, "ffn2_" + std::to_string(i),
                                                     true, true, "gpu", "xavier");
            Layers::MultiHeadAttention* m = b.mha.get();
            for (int w = 0; w < 4; ++w)
                s->params.push_back({[m, w]() -> DeviceTensor& { return m->weight(w); },
                                     [m, w]() -> DeviceTensor& { return m->grad_weight(w); }});
            Layers::BatchNorm* bn = b.bn.get();
            s->params.push_back({[bn]() -> DeviceTensor& { return bn->gamma(); },
                                 [bn]() -> DeviceTensor& { return bn->grad_gamma(); }});
            s->params.push_back({[bn]() -> DeviceTensor& { return bn->beta(); },
                                 [bn]() -> DeviceTensor& { return bn->grad_beta(); }});
            s->add_params(b.ff1);
            s->add_params(b.ff2);
            net->blocks.push_back(std::move(b));
        }
        net->pool = std::make_shared<Layers::MeanPool1D>("gpu");
        net->pool->set_row_order(CNHIP_ROWS_BY_SAMPLE);
        net->fc = std::make_shared<Layers::Linear>(D, static_cast<int>(classes), "classifier", true, true, "gpu",
                                                   "xavier");
        s->add_params(net->fc);
        s->encoder = std::move(net);
        s->loss = make_loss(CNT_LOSS_SOFTMAX_CE);
        s->opt = std::make_unique<Optimizers::Adam>(beta1, beta2, eps, "gpu");
        s->lr = lr;
        s->X = DeviceTensor::zeros({batch, seq_len});  // int32 ids
        s->Y = DeviceTensor::zeros({batch, classes});
        Device::synchronize();
        *out = s.release();
    });
}

int cnt_destroy(cnt_session* s)
{
    return guarded("cnt_destroy", [&] {
        if (!s) return;
        cnhip_stream_synchronize(s->stream);
        cnhip_stream_t st = s->stream;
        {
            StreamScope scope(s);
            release_graph(s);
            delete s;
        }
        cnhip_stream_destroy(st);
    });
}

int cnt_num_params(cnt_session* s, int* count)
{
    return guarded("cnt_num_params", [&] {
        check_session(s);
        *count = static_cast<int>(s->params.size());
    });
}

int cnt_param_size(cnt_session* s, int index, int64_t* n)
{
    return guarded("cnt_param_size", [&] { *n = param_at(s, index, false).size(); });
}

int cnt_set_param(cnt_session* s, int index, const float* host)
{
    return guarded("cnt_set_param", [&] {
        check_session(s);
        StreamScope scope(s);
        param_from_host(s, index, host);
    });
}

int cnt_get_param(cnt_session* s, int index, float* host)
{
    return guarded("cnt_get_param", [&] {
        check_session(s);
        StreamScope scope(s);
        param_to_host(s, index, false, host);
    });
}

int cnt_get_grad(cnt_session* s, int index, float* host)
{
    return guarded("cnt_get_grad", [&] {
        check_session(s);
        StreamScope scope(s);
        param_to_host(s, index, true, host);
    });
}

int cnt_get_opt_state(cnt_session* s, int index, int k, float* host, int* t)
{
    return guarded("cnt_get_opt_state", [&] {
        check_session(s);
        StreamScope scope(s);
        if (!host || !t) throw std::invalid_argument("NULL output");
        if (k < 0 || k >= s->opt->state_tensors())
            throw std::invalid_argument("state tensor " + std::to_string(k) + " of an optimizer that keeps " +
                                        std::to_string(s->opt->state_tensors()));
        auto& p = param_rec(s, index);
        DeviceTensor& w = p.value();
        std::vector<std::vector<float>> st;
        int tt = 0;
        if (!s->opt->get_state(w.data(), w.size(), st, tt)) st.assign(k + 1, std::vector<float>(w.size(), 0.f));
        *t = tt;
        const std::vector<float>& v = st[k];
        if (p.t_rows == 0)
        {
            std::copy(v.begin(), v.end(), host);
            return;
        }
        // the device keeps the transpose of the reference's [t_rows, t_cols]
        for (int64_t r = 0; r < p.t_rows; ++r)
            for (int64_t c = 0; c < p.t_cols; ++c) host[r + p.t_rows * c] = v[c + p.t_cols * r];
    });
}

namespace
{
    // The token ids of a batch are checked once, when the batch is uploaded
    // (as the cpu-eigen Embedding::forward does per call, embedding.cpp:87-90),
    // so the training steps themselves never synchronise.
    void check_token_ids(const int32_t* ids, int64_t B, int64_t S, int64_t V)
    {
        for (int64_t n = 0; n < B; ++n)
            for (int64_t t = 0; t < S; ++t)
            {
                const int32_t id = ids[n + B * t];
                if (id < 0 || id >= V)
                    throw std::out_of_range("Embedding: token ID " + std::to_string(id) + " out of range [0, " +
                                            std::to_string(V) + ")");
            }
    }
} // namespace

int cnt_set_batch_tokens(cnt_session* s, const int32_t* ids_host, const float* y_host)
{
    return guarded("cnt_set_batch_tokens", [&] {
        check_session(s);
        if (!s->encoder) throw std::invalid_argument("not a token-input (transformer) session");
        check_token_ids(ids_host, s->X.dimension(0), s->X.dimension(1), s->encoder->emb->get_vocab_size());
        StreamScope scope(s);
        s->X.copy_from_host(ids_host);
        s->Y.copy_from_host(y_host);
    });
}

int cnt_set_batch(cnt_session* s, const float* x_host, const float* y_host)
{
    return guarded("cnt_set_batch", [&] {
        check_session(s);
        if (s->encoder) throw std::invalid_argument("transformer sessions take int32 ids: use cnt_set_batch_tokens");
        StreamScope scope(s);
        s->X.copy_from_host(x_host);
        s->Y.copy_from_host(y_host);
    });
}

int cnt_set_batch_device(cnt_session* s, const float* x_dev, const float* y_dev)
{
    return guarded("cnt_set_batch_device", [&] {
        check_session(s);
        StreamScope scope(s);
        Device::check(cnhip_memcpy_async(s->X.data(), x_dev, static_cast<size_t>(s->X.size()) * 4, 2,
                                         s->stream), "X");
        Device::check(cnhip_memcpy_async(s->Y.data(), y_dev, static_cast<size_t>(s->Y.size()) * 4, 2,
                                         s->stream), "Y");
        if (s->encoder)  // token ids: one read-back here instead of one per step
        {
            std::vector<int32_t> ids(static_cast<size_t>(s->X.size()));
            s->X.copy_to_host(ids.data());
            check_token_ids(ids.data(), s->X.dimension(0), s->X.dimension(1), s->encoder->emb->get_vocab_size());
        }
    });
}

namespace
{
    void forward_backward(cnt_session* s)
    {
        if (s->encoder)
        {
            s->encoder->zero_grad();
            DeviceTensor out = s->encoder->forward(s->X);
            DeviceTensor g;
            if (auto* sce = dynamic_cast<Losses::SoftmaxCrossEntropy*>(s->loss.get()))
                s->last_loss = sce->forward_backward(out, s->Y, g);
            else if (auto* mse = dynamic_cast<Losses::MSE*>(s->loss.get()))
                s->last_loss = mse->forward_backward(out, s->Y, g);
            else
            {
                s->last_loss = s->loss->forward(out, s->Y);
                g = s->loss->backward(out, s->Y);
            }
            s->encoder->backward(g);
            return;
        }
        s->model.zero_grad();
        // A Sigmoid output step followed by BinaryCrossEntropy on a small
        // output runs as one launch (cnhip_sigmoid_bce_head), bit-identical
        // to the four separate ones.
        auto* bce = dynamic_cast<Losses::BinaryCrossEntropy*>(s->loss.get());
        const std::size_t n = s->model.num_steps();
        if (bce && n >= 2 && dynamic_cast<Activations::Sigmoid*>(s->model.last_activation()) &&
            s->Y.size() <= kFusedHeadMax)
        {
            DeviceTensor z = s->model.forward_prefix(s->X, n - 1);
            if (z.dims() != s->Y.dims())
                throw std::invalid_argument("model output " + shape_str(z.dims()) + " and targets " +
                                            shape_str(s->Y.dims()) + " differ");
            DeviceTensor p = DeviceTensor::empty(z.dims()), dz = DeviceTensor::empty(z.dims());
            DeviceTensor loss = DeviceTensor::empty({1});
            Device::check(cnhip_sigmoid_bce_head(z.data(), s->Y.data(), p.data(), loss.data(), dz.data(), z.size(),
                                                 bce->forward_reduction(), bce->backward_reduction(), s->stream),
                          "sigmoid + BCE head");
            s->last_loss = Losses::DeviceScalar(loss);
            s->model.backward_params_prefix(dz, n - 1);
            return;
        }
        DeviceTensor out = s->model.forward(s->X);
        DeviceTensor g;
        if (auto* sce = dynamic_cast<Losses::SoftmaxCrossEntropy*>(s->loss.get()))
            s->last_loss = sce->forward_backward(out, s->Y, g);  // one launch for small batches
        else if (auto* mse = dynamic_cast<Losses::MSE*>(s->loss.get()))
            s->last_loss = mse->forward_backward(out, s->Y, g);  // one launch for small outputs
        else
        {
            s->last_loss = s->loss->forward(out, s->Y);
            g = s->loss->backward(out, s->Y);
        }
        s->model.backward_params(g);
    }

    // Eager forward + backward.  The layers' host-side state (cached
    // activations, argmax indices) then belongs to this pass, so a captured
    // graph, whose replays would not update it, is dropped first.
    void eager_forward_backward(cnt_session* s)
    {
        release_graph(s);
        forward_backward(s);
        s->warm = true;
    }

    // The whole step of Linear(I, H) -> ReLU -> Linear(H, 1) -> Sigmoid with
    // BinaryCrossEntropy and Adam (config 1's model) in two launches
    // (cnhip_mlp2_bce_adam_step) instead of seven: at its sizes the host's
    // issue time per launch exceeded the GPU's work.  Taken while no graph
    // is captured; false where it does not apply.  The layers' forward caches
    // are not written (nothing after a full step reads them; the split calls
    // and a capture run their own forward); the gradients are this step's.
    bool fused_mlp_step(cnt_session* s)
    {
        if (!s->fused_steps || s->encoder || s->graph || s->model.num_steps() != 4) return false;
        auto* adam = dynamic_cast<Optimizers::Adam*>(s->opt.get());
        auto* bce = dynamic_cast<Losses::BinaryCrossEntropy*>(s->loss.get());
        Layers::Linear* l1 = s->model.step_linear(0);
        Layers::Linear* l2 = s->model.step_linear(2);
        if (!adam || !bce || !l1 || !l2 || !dynamic_cast<Activations::ReLU*>(s->model.step_activation(1)) ||
            !dynamic_cast<Activations::Sigmoid*>(s->model.step_activation(3)) || !l1->is_trainable() ||
            !l2->is_trainable())
            return false;
        const int64_t I = l1->get_input_size(), H = l1->get_output_size();
        if (s->X.dims().size() != 2 || s->X.dimension(1) != I || l2->get_input_size() != H ||
            l2->get_output_size() != 1 || I > 64 || H > 64)
            return false;
        const int64_t B = s->X.dimension(0);
        if (B % 16 != 0 || B / 16 > 65535 || s->Y.size() != B) return false;
        DeviceTensor& W1 = l1->weights();
        DeviceTensor& b1 = l1->biases();
        DeviceTensor& W2 = l2->weights();
        DeviceTensor& b2 = l2->biases();
        DeviceTensor& gW1 = l1->grad_weights();
        DeviceTensor& gb1 = l1->grad_biases();
        DeviceTensor& gW2 = l2->grad_weights();
        DeviceTensor& gb2 = l2->grad_biases();
        std::vector<float*> m, v;
        std::vector<float> bc1, bc2;
        adam->prepare_external({{W1.data(), W1.size()}, {b1.data(), b1.size()}, {W2.data(), W2.size()},
                                {b2.data(), b2.size()}},
                               m, v, bc1, bc2);
        DeviceTensor loss;
        int st = CNHIP_OK;
        try
        {
            loss = DeviceTensor::empty({1});
            st = cnhip_mlp2_bce_adam_step(s->X.data(), s->Y.data(), B, I, H, W1.data(), b1.data(), W2.data(),
                                          b2.data(), gW1.data(), gb1.data(), gW2.data(), gb2.data(), m.data(),
                                          v.data(), bc1.data(), bc2.data(), s->lr, adam->beta1(), adam->beta2(),
                                          adam->epsilon(), bce->forward_reduction(), bce->backward_reduction(),
                                          loss.data(), s->stream);
        }
        catch (...)
        {
            adam->abort_external();
            throw;
        }
        if (st != CNHIP_OK)
        {
            adam->abort_external();  // nothing was updated: the step counts go back
            Device::check(st, "fused MLP step");
        }
        adam->commit_external();
        s->fused_taken = true;
        l1->set_grads_pending_zero(false);
        l2->set_grads_pending_zero(false);
        s->last_loss = Losses::DeviceScalar(loss);
        s->updated = true;
        return true;
    }

    void update(cnt_session* s)
    {
        if (s->encoder)
            s->encoder->update(*s->opt, s->lr);
        else
            s->model.update(*s->opt, s->lr);
        s->updated = true;
    }

    // A persistent recurrence launch that gave up waiting leaves invalid
    // outputs; the device then withholds every optimizer launch queued after
    // it.  Taking the fault (at a sync point, or when the next recurrent call
    // or graph replay finds it) reports it here, after the optimizer's step
    // counts of the withheld updates are rolled back: parameters and
    // optimizer state are then as before the faulted step.
    void take_recurrence_fault(cnt_session* s, const char* who)
    {
        const int st = cnhip_recurrence_fault_check(s->stream);
        if (s->opt) s->opt->reconcile_withheld();
        Device::check(st, who);
    }

    // Runs f; on an error, first rolls back what a fault taken inside it withheld.
    void reconciled(cnt_session* s, const std::function<void()>& f)
    {
        try
        {
            f();
        }
        catch (...)
        {
            if (s->opt) s->opt->reconcile_withheld();
            throw;
        }
    }
} // namespace

namespace
{
    std::vector<Layers::Layer*> file_layers(cnt_session* s)
    {
        check_session(s);
        return s->all_layers();
    }

    const char* check_path(const char* path)
    {
        if (!path || !*path) throw std::invalid_argument("empty path");
        return path;
    }
} // namespace

int cnt_save_model(cnt_session* s, const char* path)
{
    return guarded("cnt_save_model", [&] {
        check_session(s);
        StreamScope scope(s);
        Utils::save_layers(check_path(path), file_layers(s), nullptr, false);
    });
}

int cnt_load_model(cnt_session* s, const char* path)
{
    return guarded("cnt_load_model", [&] {
        check_session(s);
        StreamScope scope(s);
        Utils::load_layers(check_path(path), file_layers(s), nullptr, false);
        Device::synchronize();
    });
}

int cnt_save_checkpoint(cnt_session* s, const char* path)
{
    return guarded("cnt_save_checkpoint", [&] {
        check_session(s);
        StreamScope scope(s);
        Utils::save_layers(check_path(path), file_layers(s), s->opt.get(), true);
    });
}

int cnt_load_checkpoint(cnt_session* s, const char* path)
{
    return guarded("cnt_load_checkpoint", [&] {
        check_session(s);
        StreamScope scope(s);
        Utils::load_layers(check_path(path), file_layers(s), s->opt.get(), true);
        Device::synchronize();
        s->updated = true;  // the optimizer now holds state: no swap after this
    });
}

struct cnt_loader
{
    std::unique_ptr<Utils::DataLoader> dl;
    int64_t F = 0, L = 0;
};

namespace
{
    Utils::DataLoader& loader_of(cnt_loader* ld)
    {
        if (!ld || !ld->dl) throw std::invalid_argument("NULL loader");
        return *ld->dl;
    }
} // namespace

int cnt_loader_create(cnt_loader** out, const float* features, const float* labels, int64_t n, int64_t f,
                      int64_t l, int64_t batch, int shuffle, int drop_last, uint64_t seed)
{
    return guarded("cnt_loader_create", [&] {
        if (!out) throw std::invalid_argument("NULL out pointer");
        *out = nullptr;
        if (n < 0 || f <= 0 || l <= 0 || n > INT32_MAX || batch > INT32_MAX)
            throw std::invalid_argument("bad dataset shape");
        if (n > 0 && (!features || !labels)) throw std::invalid_argument("NULL data");
        Tensor<float, 2> X(n, f), Y(n, l);
        if (n) std::copy(features, features + n * f, X.data());
        if (n) std::copy(labels, labels + n * l, Y.data());
        auto ld = std::make_unique<cnt_loader>();
        ld->dl = std::make_unique<Utils::DataLoader>(std::move(X), std::move(Y), static_cast<int>(batch), shuffle != 0,
                                                     drop_last != 0);
        ld->dl->set_seed(seed);
        ld->F = f;
        ld->L = l;
        *out = ld.release();
    });
}

int cnt_loader_destroy(cnt_loader* ld)
{
    return guarded("cnt_loader_destroy", [&] { delete ld; });
}

int cnt_loader_num_batches(cnt_loader* ld, int64_t* count)
{
    return guarded("cnt_loader_num_batches", [&] {
        if (!count) throw std::invalid_argument("NULL out pointer");
        *count = static_cast<int64_t>(loader_of(ld).num_batches());
    });
}

int cnt_loader_indices(cnt_loader* ld, int32_t* out)
{
    return guarded("cnt_loader_indices", [&] {
        const auto& v = loader_of(ld).indices();
        if (!v.empty() && !out) throw std::invalid_argument("NULL out pointer");
        std::copy(v.begin(), v.end(), out);
    });
}

int cnt_loader_reset(cnt_loader* ld)
{
    return guarded("cnt_loader_reset", [&] { loader_of(ld).reset(); });
}

int cnt_loader_host_batch(cnt_loader* ld, int64_t k, float* x, float* y, int64_t* bs)
{
    return guarded("cnt_loader_host_batch", [&] {
        if (!x || !y || !bs) throw std::invalid_argument("NULL argument");
        if (k < 0) throw std::out_of_range("DataLoader: batch index out of range");
        Utils::Batch b = loader_of(ld).get_batch(static_cast<std::size_t>(k));
        *bs = b.features.dimension(0);
        std::copy(b.features.data(), b.features.data() + b.features.size(), x);
        std::copy(b.labels.data(), b.labels.data() + b.labels.size(), y);
    });
}

int cnt_loader_to_device(cnt_loader* ld, int mode)
{
    return guarded("cnt_loader_to_device", [&] {
        if (mode != CNT_STAGE_RESIDENT && mode != CNT_STAGE_STREAM)
            throw std::invalid_argument("mode must be CNT_STAGE_RESIDENT or CNT_STAGE_STREAM");
        loader_of(ld).to_device(mode == CNT_STAGE_RESIDENT ? Utils::Staging::Resident : Utils::Staging::Stream);
    });
}

int cnt_loader_next(cnt_loader* ld, float* x_dev, float* y_dev, int64_t* bs, void* stream)
{
    return guarded("cnt_loader_next", [&] {
        if (!bs) throw std::invalid_argument("NULL bs");
        Utils::DataLoader& dl = loader_of(ld);
        const cnhip_stream_t saved = Device::stream();
        Device::set_stream(static_cast<cnhip_stream_t>(stream));
        try
        {
            *bs = dl.next_into(x_dev, y_dev);
        }
        catch (...)
        {
            Device::set_stream(saved);
            throw;
        }
        Device::set_stream(saved);
    });
}

int cnt_loader_next_batch(cnt_loader* ld, cnt_session* s, int64_t* bs)
{
    return guarded("cnt_loader_next_batch", [&] {
        check_session(s);
        if (!bs) throw std::invalid_argument("NULL bs");
        Utils::DataLoader& dl = loader_of(ld);
        if (s->encoder) throw std::invalid_argument("token-id sessions take cnt_set_batch_tokens");
        const int64_t next = dl.next_size();
        *bs = 0;
        if (next == 0) return;
        if (s->X.dimension(0) != next || s->X.size() != next * ld->F || s->Y.size() != next * ld->L)
            throw std::invalid_argument("the loader's next batch is " + std::to_string(next) + " x (" +
                                        std::to_string(ld->F) + ", " + std::to_string(ld->L) +
                                        ") but the session's batch is X " + shape_str(s->X.dims()) + ", Y " +
                                        shape_str(s->Y.dims()) + " (use drop_last or a dividing batch size)");
        StreamScope scope(s);
        *bs = dl.next_into(s->X.data(), s->Y.data());
    });
}

int cnt_npy_save(const char* path, const float* colmajor, int ndims, const int64_t* dims)
{
    return guarded("cnt_npy_save", [&] {
        if (ndims < 1 || !dims) throw std::invalid_argument("rank must be at least 1");
        int64_t n = 1;
        for (int i = 0; i < ndims; ++i) n *= dims[i];
        if (n > 0 && !colmajor) throw std::invalid_argument("NULL data");
        Utils::save_npy_raw(check_path(path), colmajor, std::vector<int64_t>(dims, dims + ndims));
    });
}

int cnt_npy_load(const char* path, float* out, int64_t capacity, int* ndims, int64_t* dims, int raw_colmajor)
{
    return guarded("cnt_npy_load", [&] {
        if (!ndims || !dims) throw std::invalid_argument("NULL ndims or dims");
        std::vector<int64_t> d;
        std::vector<float> v = Utils::load_npy_raw(check_path(path), d, raw_colmajor != 0);
        if (static_cast<int>(d.size()) > *ndims)
            throw std::invalid_argument("the file's rank " + std::to_string(d.size()) + " exceeds the dims capacity");
        if (static_cast<int64_t>(v.size()) > capacity || (!v.empty() && !out))
            throw std::invalid_argument("the file holds " + std::to_string(v.size()) + " floats, capacity " +
                                        std::to_string(capacity));
        *ndims = static_cast<int>(d.size());
        for (std::size_t i = 0; i < d.size(); ++i) dims[i] = d[i];
        if (!v.empty()) std::copy(v.begin(), v.end(), out);
    });
}

int cnt_set_optimizer(cnt_session* s, int kind, float hyper, float eps)
{
    return guarded("cnt_set_optimizer", [&] {
        check_session(s);
        if (s->updated) throw std::logic_error("the session has already updated its parameters");
        StreamScope scope(s);
        switch (kind)
        {
            case CNT_OPT_ADAM: s->opt = std::make_unique<Optimizers::Adam>(hyper, 0.999f, eps, "gpu"); break;
            case CNT_OPT_SGD: s->opt = std::make_unique<Optimizers::SGD>("gpu"); break;
            case CNT_OPT_MOMENTUM: s->opt = std::make_unique<Optimizers::Momentum>(hyper, "gpu"); break;
            case CNT_OPT_ADAGRAD: s->opt = std::make_unique<Optimizers::Adagrad>(eps, "gpu"); break;
            case CNT_OPT_RMSPROP: s->opt = std::make_unique<Optimizers::RMSProp>(hyper, eps, "gpu"); break;
            default: throw std::invalid_argument("unknown optimizer code " + std::to_string(kind));
        }
    });
}

int cnt_step(cnt_session* s, float* loss_out)
{
    return guarded("cnt_step", [&] {
        check_session(s);
        StreamScope scope(s);
        take_recurrence_fault(s, "cnt_step");  // one left by an earlier step
        reconciled(s, [&] {
            if (s->graph)
            {
                Device::check(cnhip_graph_launch(s->graph, s->stream), "cnt_step graph replay");
                s->last_loss = s->graph_loss;
                for (auto& f : s->graph_flags) f.first->set_grads_pending_zero(f.second);
            }
            else if (fused_mlp_step(s))
                return;
            else
                eager_forward_backward(s);
            update(s);
        });
        if (loss_out)
        {
            *loss_out = s->last_loss.get();
            take_recurrence_fault(s, "cnt_step");  // this step's, now that it has run
        }
    });
}

int cnt_set_fused_step(cnt_session* s, int enable)
{
    return guarded("cnt_set_fused_step", [&] {
        check_session(s);
        s->fused_steps = enable != 0;
    });
}

int cnt_capture_step(cnt_session* s)
{
    return guarded("cnt_capture_step", [&] {
        check_session(s);
        StreamScope scope(s);
        release_graph(s);
        // after fused steps only, one eager layer-by-layer forward + backward
        // (no update) sizes what the graph's kernels refer to
        if (!s->warm && s->fused_taken) eager_forward_backward(s);
        if (!s->warm)
            throw std::logic_error("run one step eagerly before capturing: it sizes the buffers and "
                                   "workspaces the graph will refer to");
        // A Dropout layer's mask position advances on the host every forward;
        // a replayed graph would repeat the captured step's masks.
        for (Layers::Layer* l : s->all_layers())
            if (dynamic_cast<Layers::Dropout*>(l))
                throw std::logic_error("a model with Dropout cannot be captured: each step draws new masks");
        Device::check(cnhip_graph_begin_capture(s->stream), "capture");
        s->graph_pool = Device::open_pool();
        cnhip_graph_t g = nullptr;
        try
        {
            forward_backward(s);
        }
        catch (...)
        {
            Device::close_pool();
            cnhip_graph_end_capture(s->stream, 0, &g);
            Device::release_pool(s->graph_pool);
            s->graph_pool = 0;
            s->warm = false;  // host-side layer state refers to work that never ran
            throw;
        }
        Device::close_pool();
        const int st = cnhip_graph_end_capture(s->stream, 1, &g);
        if (st != CNHIP_OK)
        {
            Device::release_pool(s->graph_pool);
            s->graph_pool = 0;
            s->warm = false;
            Device::check(st, "capture");
        }
        s->graph = g;
        s->graph_loss = s->last_loss;
        for (Layers::Layer* l : s->all_layers()) s->graph_flags.emplace_back(l, l->grads_pending_zero());
    });
}

int cnt_release_graph(cnt_session* s)
{
    return guarded("cnt_release_graph", [&] {
        check_session(s);
        StreamScope scope(s);
        release_graph(s);
    });
}

int cnt_has_graph(cnt_session* s) { return s && s->graph ? 1 : 0; }

int cnt_forward_backward(cnt_session* s, float* loss_out)
{
    return guarded("cnt_forward_backward", [&] {
        check_session(s);
        StreamScope scope(s);
        take_recurrence_fault(s, "cnt_forward_backward");
        reconciled(s, [&] { eager_forward_backward(s); });
        if (loss_out)
        {
            *loss_out = s->last_loss.get();
            take_recurrence_fault(s, "cnt_forward_backward");
        }
    });
}

int cnt_update(cnt_session* s)
{
    return guarded("cnt_update", [&] {
        check_session(s);
        StreamScope scope(s);
        take_recurrence_fault(s, "cnt_update");
        reconciled(s, [&] { update(s); });
    });
}

int cnt_synchronize(cnt_session* s)
{
    return guarded("cnt_synchronize", [&] {
        check_session(s);
        Device::check(cnhip_stream_synchronize(s->stream), "sync");
        take_recurrence_fault(s, "cnt_synchronize");
    });
}

void* cnt_stream(cnt_session* s) { return s ? s->stream : nullptr; }

} // extern "C"
