// Training harness C ABI (include/cppnet_train.h): builds models from the
// CppNet-compatible classes and runs the reference harness's train step.
#include "cppnet_train.h"

#include <cstdarg>
#include <cstdio>
#include <exception>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "CppNet/CppNet.hpp"

using namespace CppNet;

struct cnt_session
{
    cnhip_stream_t stream = nullptr;
    Models::SequentialModel model;
    std::vector<std::shared_ptr<Layers::Layer>> keep;  // owns the layers
    std::unique_ptr<Losses::Loss> loss;
    std::unique_ptr<Optimizers::Adam> adam;
    float lr = 1e-3f;
    DeviceTensor X, Y;
    Losses::DeviceScalar last_loss;

    // parameter index -> accessors of the value and of the gradient, called
    // through the layer so lazily-zeroed gradients are materialised first
    struct Param
    {
        std::function<DeviceTensor&()> value, grad;
    };
    std::vector<Param> params;

    template <class L>
    void add_params(const std::shared_ptr<L>& l)
    {
        L* p = l.get();
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
        }
        throw std::invalid_argument("unknown loss code " + std::to_string(loss));
    }

    void check_session(cnt_session* s)
    {
        if (!s) throw std::invalid_argument("NULL session");
    }

    DeviceTensor& param_at(cnt_session* s, int index, bool grad)
    {
        check_session(s);
        if (index < 0 || index >= static_cast<int>(s->params.size()))
            throw std::out_of_range("parameter index " + std::to_string(index) + " out of range");
        auto& p = s->params[static_cast<size_t>(index)];
        return grad ? p.grad() : p.value();
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
    return guarded("cnt_mlp_create", [&] {
        if (!out) throw std::invalid_argument("NULL out pointer");
        *out = nullptr;
        if (n_linear < 1 || !sizes) throw std::invalid_argument("need at least one Linear layer");
        if (batch <= 0) throw std::invalid_argument("batch must be positive");
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
        }
        s->loss = make_loss(loss);
        s->adam = std::make_unique<Optimizers::Adam>(beta1, beta2, eps, "gpu");
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
        s->adam = std::make_unique<Optimizers::Adam>(beta1, beta2, eps, "gpu");
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
        else
            throw std::invalid_argument("cell must be 0 (LSTM) or 1 (GRU)");
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
        s->adam = std::make_unique<Optimizers::Adam>(beta1, beta2, eps, "gpu");
        s->lr = lr;
        s->X = DeviceTensor::zeros({batch, seq_len, input_size});
        s->Y = DeviceTensor::zeros({batch, out_features});
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
        StreamScope scope(s);
        param_at(s, index, false).copy_from_host(host);
    });
}

int cnt_get_param(cnt_session* s, int index, float* host)
{
    return guarded("cnt_get_param", [&] {
        StreamScope scope(s);
        param_at(s, index, false).copy_to_host(host);
    });
}

int cnt_get_grad(cnt_session* s, int index, float* host)
{
    return guarded("cnt_get_grad", [&] {
        StreamScope scope(s);
        param_at(s, index, true).copy_to_host(host);
    });
}

int cnt_set_batch(cnt_session* s, const float* x_host, const float* y_host)
{
    return guarded("cnt_set_batch", [&] {
        check_session(s);
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
    });
}

namespace
{
    void forward_backward(cnt_session* s)
    {
        s->model.zero_grad();
        DeviceTensor out = s->model.forward(s->X);
        s->last_loss = s->loss->forward(out, s->Y);
        DeviceTensor g = s->loss->backward(out, s->Y);
        s->model.backward(g);
    }
} // namespace

int cnt_step(cnt_session* s, float* loss_out)
{
    return guarded("cnt_step", [&] {
        check_session(s);
        StreamScope scope(s);
        forward_backward(s);
        s->model.update(*s->adam, s->lr);
        if (loss_out) *loss_out = s->last_loss.get();
    });
}

int cnt_forward_backward(cnt_session* s, float* loss_out)
{
    return guarded("cnt_forward_backward", [&] {
        check_session(s);
        StreamScope scope(s);
        forward_backward(s);
        if (loss_out) *loss_out = s->last_loss.get();
    });
}

int cnt_update(cnt_session* s)
{
    return guarded("cnt_update", [&] {
        check_session(s);
        StreamScope scope(s);
        s->model.update(*s->adam, s->lr);
    });
}

int cnt_synchronize(cnt_session* s)
{
    return guarded("cnt_synchronize", [&] {
        check_session(s);
        Device::check(cnhip_stream_synchronize(s->stream), "sync");
    });
}

void* cnt_stream(cnt_session* s) { return s ? s->stream : nullptr; }

} // extern "C"
