"""The public C++ API compiles and links the way a CppNet program would use it
(no GPU needed: the program is built, not run).  The program touches every
class family the headers declare -- layers, activations, losses, optimizers,
the model, the DataLoader and the model-file functions -- with the
reference's constructor arguments."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "cppnet_amd" / "_lib"

PROGRAM = r'''
#include <CppNet/CppNet.hpp>
#include <memory>
using namespace CppNet;

int main(int argc, char**) {
    if (argc < 100) return 0;  // built to check the API; never executed
    Models::SequentialModel model;
    model.add_layer(std::make_shared<Layers::Linear>(30, 64, "fc1", true, true, "gpu", "xavier"));
    model.add_activation(std::make_shared<Activations::LeakyReLU>(0.01f, "gpu"));
    model.add_layer(std::make_shared<Layers::Linear>(64, 10, "fc2", true, true, "gpu", "xavier"));
    model.add_activation(std::make_shared<Activations::Softmax>("gpu"));
    Layers::Conv2D conv(3, 8, 3, 1, 1, true, "gpu");
    Layers::MaxPool2D pool(2, 2, "gpu");
    Layers::GlobalAvgPool2D gap("gpu");
    Layers::GlobalMaxPool2D gmp("gpu");
    Layers::Dropout drop(0.5f, "gpu");
    Layers::LSTM lstm(8, 16, true, "gpu");
    Layers::GRU gru(8, 16, true, "gpu");
    Layers::RNN rnn(8, 16, true, "gpu");
    Layers::MultiHeadAttention mha(32, 4, "gpu");
    Layers::BatchNorm bn(32, 0.1f, 1e-5f, "gpu");
    Layers::Embedding emb(100, 32, "gpu");
    Losses::CategoricalCrossEntropy cce("mean", true, 0.1f, "gpu");
    Losses::MAE mae("mean", "gpu");
    Losses::Huber huber(1.0f, "mean", "gpu");
    Losses::SoftmaxCrossEntropy sce("mean", "gpu");
    Optimizers::Adam adam;
    Optimizers::SGD sgd("gpu");
    Optimizers::Momentum mom(0.9f, "gpu");
    Optimizers::Adagrad ada(1e-8f, "gpu");
    Optimizers::RMSProp rms(0.9f, 1e-8f, "gpu");
    Tensor<float, 2> X(100, 30), Y(100, 10);
    Utils::DataLoader loader(X, Y, 32, true, false);
    loader.to_device(Utils::Staging::Resident);
    Utils::DeviceBatch batch;
    while (loader.next_device(batch)) {
        model.zero_grad();
        DeviceTensor out = model.forward(batch.features);
        float l = cce.forward(out, batch.labels).get();
        model.backward_params(cce.backward(out, batch.labels));
        model.update(rms, 1e-3f);
        (void)l;
    }
    for (auto b : loader) (void)b;
    Utils::save_model("m.cnet", model);
    Utils::load_model("m.cnet", model);
    Utils::save_checkpoint("m.ckpt", model, &rms);
    Utils::load_checkpoint("m.ckpt", model, &rms);
    Utils::save_npy("x.npy", X);
    Tensor<float, 2> x2 = Utils::load_npy_2d("x.npy");
    return static_cast<int>(x2.size() + conv.get_out_channels() + sgd.get_gpu_block_size());
}
'''


@pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")
def test_public_headers_compile_and_link(tmp_path):
    if not (LIB / "libcppnet.so").exists():
        pytest.skip("libraries not built (python -m cppnet_amd.build)")
    src = tmp_path / "app.cpp"
    src.write_text(PROGRAM)
    cmd = ["g++", "-std=c++17", "-Wall", "-Werror", "-Wno-unused-variable", f"-I{ROOT / 'cppnet_amd' / 'include'}",
           f"-I{ROOT / 'include'}", str(src), f"-L{LIB}", "-lcppnet", "-lcnhip", f"-Wl,-rpath,{LIB}",
           "-o", str(tmp_path / "app")]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-4000:]


# Reference code that writes through a state getter (the reference returns
# mutable references, e.g. batch_norm.hpp:74-77, linear.hpp:81, and its own
# load_model does `bn->get_gamma() = read_tensor_1d(ifs)`,
# serialization.cpp:238-239).  Here the getters return host copies of HBM
# state, so each such write must be a compile error, never a silent no-op.
WRITE_THROUGH_GETTER = {
    "assign_gamma": "Tensor<float, 1> g(4); bn.get_gamma() = g;",
    "assign_beta": "Tensor<float, 1> g(4); bn.get_beta() = g;",
    "assign_running_var": "Tensor<float, 1> g(4); bn.get_running_var() = g;",
    "element_write_weights": "lin.get_weights()(0, 0) = 1.0f;",
    "element_write_biases": "lin.get_biases()(0) = 1.0f;",
    "setzero_conv_weights": "conv.get_weights().setZero();",
    "bind_mutable_ref": "Tensor<float, 2>& w = lin.get_weights(); w(0, 0) = 1.0f;",
    "assign_lstm_whh": "Tensor<float, 2> w(4, 16); lstm.get_W_hh() = w;",
    "assign_embedding": "Tensor<float, 2> w(10, 4); emb.get_weight() = w;",
    "assign_mha_weight": "Tensor<float, 2> w(4, 4); mha.get_weight(0) = w;",
}

GETTER_PROGRAM = r'''
#include <CppNet/CppNet.hpp>
using namespace CppNet;
void f(Layers::BatchNorm& bn, Layers::Linear& lin, Layers::Conv2D& conv, Layers::LSTM& lstm,
       Layers::Embedding& emb, Layers::MultiHeadAttention& mha) {
    (void)bn; (void)lin; (void)conv; (void)lstm; (void)emb; (void)mha;
    BODY
}
'''

# What such code must do instead: copy, modify, set back.
SETTER_BODY = ("Tensor<float, 1> g = bn.get_gamma(); g(0) = 2.0f; bn.set_gamma(g);"
               " auto w = lin.get_weights(); w(0, 0) = 1.0f; lin.set_weights(w);"
               " const auto& r = bn.get_running_mean(); (void)r;")


def _syntax_check(tmp_path, name, body):
    src = tmp_path / f"{name}.cpp"
    src.write_text(GETTER_PROGRAM.replace("BODY", body))
    cmd = ["g++", "-std=c++17", "-fsyntax-only", f"-I{ROOT / 'cppnet_amd' / 'include'}",
           f"-I{ROOT / 'include'}", str(src)]
    return subprocess.run(cmd, capture_output=True, text=True, timeout=300)


@pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")
@pytest.mark.parametrize("case", sorted(WRITE_THROUGH_GETTER))
def test_write_through_getter_fails_to_compile(tmp_path, case):
    res = _syntax_check(tmp_path, case, WRITE_THROUGH_GETTER[case])
    assert res.returncode != 0, f"{case} compiled: a write through a getter would be silently lost"
    assert "error" in res.stderr


@pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")
def test_copy_modify_set_compiles(tmp_path):
    res = _syntax_check(tmp_path, "setter", SETTER_BODY)
    assert res.returncode == 0, res.stderr[-4000:]
