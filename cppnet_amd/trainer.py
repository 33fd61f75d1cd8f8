"""ctypes front end of the C++ training harness (include/cppnet_train.h).

A Session is a model built by libcppnet.so from the CppNet-compatible layer
classes on device "gpu"; every step runs in C++/HIP.  The helpers here only
describe the benchmark configurations and generate their synthetic data.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _capi

ACT = {"none": 0, "relu": 1, "sigmoid": 2, "tanh": 3, "leaky_relu": 4, "softmax": 5}
LOSS = {"bce": 0, "softmax_ce": 1, "mse": 2, "cce": 3, "mae": 4, "huber": 5}
OPT = {"adam": 0, "sgd": 1, "momentum": 2, "adagrad": 3, "rmsprop": 4}
CELL = {"lstm": 0, "gru": 1, "rnn": 2}
GATES = {"lstm": 4, "gru": 3, "rnn": 1}

_lib = None


def load() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    _capi.load()  # libcnhip.so first (RTLD_GLOBAL)
    path = _capi.LIBDIR / "libcppnet.so"
    if not path.exists():
        raise ImportError(f"{path} is missing: run `python -m cppnet_amd.build` first")
    lib = C.CDLL(str(path))
    vp, i32, i64, f32 = C.c_void_p, C.c_int, C.c_int64, C.c_float
    sigs = {
        "cnt_last_error": (C.c_char_p, []),
        "cnt_mlp_create": (i32, [C.POINTER(vp), i32, C.POINTER(i64), i32, i32, i32, i64, f32, f32,
                                 f32, f32, C.c_uint64]),
        "cnt_mlp_create_ex": (i32, [C.POINTER(vp), i32, C.POINTER(i64), i32, i32, i32, i64, f32, f32,
                                    f32, f32, C.c_uint64, f32]),
        "cnt_cnn_create": (i32, [C.POINTER(vp), i32, C.POINTER(i64), i32, C.POINTER(i64), i64, f32,
                                 f32, f32, f32, C.c_uint64]),
        "cnt_rnn_create": (i32, [C.POINTER(vp), i32, i64, i64, i64, i64, i64, f32, f32, f32, f32,
                                 C.c_uint64]),
        "cnt_transformer_create": (i32, [C.POINTER(vp), i64, i64, i64, i64, i64, i32, i64, i64, f32,
                                         f32, f32, f32, C.c_uint64]),
        "cnt_resnet_create": (i32, [C.POINTER(vp), i64, i64, i32, i64, i64, i64, f32, f32, f32, f32,
                                    C.c_uint64]),
        "cnt_set_batch_tokens": (i32, [vp, vp, vp]),
        "cnt_destroy": (i32, [vp]),
        "cnt_set_optimizer": (i32, [vp, i32, f32, f32]),
        "cnt_save_model": (i32, [vp, C.c_char_p]),
        "cnt_load_model": (i32, [vp, C.c_char_p]),
        "cnt_save_checkpoint": (i32, [vp, C.c_char_p]),
        "cnt_load_checkpoint": (i32, [vp, C.c_char_p]),
        "cnt_loader_create": (i32, [C.POINTER(vp), vp, vp, i64, i64, i64, i64, i32, i32, C.c_uint64]),
        "cnt_loader_destroy": (i32, [vp]),
        "cnt_loader_num_batches": (i32, [vp, C.POINTER(i64)]),
        "cnt_loader_indices": (i32, [vp, vp]),
        "cnt_loader_reset": (i32, [vp]),
        "cnt_loader_host_batch": (i32, [vp, i64, vp, vp, C.POINTER(i64)]),
        "cnt_loader_to_device": (i32, [vp, i32]),
        "cnt_loader_next": (i32, [vp, vp, vp, C.POINTER(i64), vp]),
        "cnt_loader_next_batch": (i32, [vp, vp, C.POINTER(i64)]),
        "cnt_npy_save": (i32, [C.c_char_p, vp, i32, C.POINTER(i64)]),
        "cnt_npy_load": (i32, [C.c_char_p, vp, i64, C.POINTER(i32), C.POINTER(i64), i32]),
        "cnt_num_params": (i32, [vp, C.POINTER(i32)]),
        "cnt_param_size": (i32, [vp, i32, C.POINTER(i64)]),
        "cnt_set_param": (i32, [vp, i32, vp]),
        "cnt_get_param": (i32, [vp, i32, vp]),
        "cnt_get_grad": (i32, [vp, i32, vp]),
        "cnt_get_opt_state": (i32, [vp, i32, i32, vp, C.POINTER(i32)]),
        "cnt_set_batch": (i32, [vp, vp, vp]),
        "cnt_set_batch_device": (i32, [vp, vp, vp]),
        "cnt_step": (i32, [vp, C.POINTER(f32)]),
        "cnt_forward_backward": (i32, [vp, C.POINTER(f32)]),
        "cnt_update": (i32, [vp]),
        "cnt_synchronize": (i32, [vp]),
        "cnt_stream": (vp, [vp]),
        "cnt_set_fused_step": (i32, [vp, i32]),
        "cnt_capture_step": (i32, [vp]),
        "cnt_release_graph": (i32, [vp]),
        "cnt_has_graph": (i32, [vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    _lib = lib
    return lib


def _check(st: int) -> None:
    if st != 0:
        raise _capi.CnhipError(f"cppnet_train status {st}: "
                               f"{load().cnt_last_error().decode(errors='replace')}")


@dataclass
class MLPConfig:
    name: str
    sizes: list
    hidden_act: str
    out_act: str
    loss: str
    batch: int
    lr: float = 1e-3
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    seed: int = 1234
    extra: dict = field(default_factory=dict)
    optimizer: str = "adam"   # OPT key; "adam" uses beta1/beta2/eps above
    opt_hyper: float = 0.9    # Momentum's mu / RMSProp's rho
    opt_eps: float = 1e-8     # Adagrad's / RMSProp's epsilon
    dropout: float = 0.0      # Dropout(p) after every hidden activation when > 0


def mlp_config(config: int, batch: int | None = None) -> MLPConfig:
    """BASELINE.json configs 1 and 2 (numbered from 1)."""
    if config == 1:
        c = MLPConfig("C1 MLP 30-64-1 sigmoid BCE", [30, 64, 1], "relu", "sigmoid", "bce", 512)
    elif config == 2:
        c = MLPConfig("C2 MLP 1024-4096-4096-10 softmax-CE", [1024, 4096, 4096, 10], "relu",
                      "none", "softmax_ce", 4096)
    else:
        raise ValueError(f"config {config} is not an MLP config")
    if batch is not None:
        c.batch = batch
    return c


@dataclass
class CNNConfig:
    """n conv blocks (in, out, kernel, stride, padding) -> ReLU -> MaxPool(pool),
    then Flatten -> Linear -> softmax-CE; input [N, C, H, W]."""
    name: str
    convs: list
    pool: int
    input_shape: list
    classes: int
    lr: float = 1e-3
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    seed: int = 1234
    loss: str = "softmax_ce"

    @property
    def batch(self) -> int:
        return self.input_shape[0]

    def flat_features(self) -> int:
        C, H, W = self.input_shape[1:]
        for (_, oc, k, s, p) in self.convs:
            H = ((H + 2 * p - k) // s + 1 - self.pool) // self.pool + 1
            W = ((W + 2 * p - k) // s + 1 - self.pool) // self.pool + 1
            C = oc
        return C * H * W


def cnn_config(config: int = 3, batch: int | None = None) -> CNNConfig:
    """Conv 3->32 (3x3, s1, p1) -> ReLU -> MaxPool 2 ->
    Conv 32->64 -> ReLU -> MaxPool 2 -> Flatten (4096) -> Linear 4096->10."""
    if config != 3:
        raise ValueError(f"config {config} is not the CNN config")
    B = 256 if batch is None else batch
    return CNNConfig("C3 CNN 2x(conv3x3, ReLU, pool2) -> 4096->10", [(3, 32, 3, 1, 1),
                     (32, 64, 3, 1, 1)], 2, [B, 3, 32, 32], 10)


def synthetic_cnn(cfg: CNNConfig, rng: np.random.Generator):
    """Conv weights xavier-uniform with fans C*k^2 / OC*k^2 (conv2d.cpp:42-50),
    biases 0; Linear xavier; X ~ U(0,1) [N,C,H,W]; one-hot uniform labels.
    All ColMajor flat float32."""
    params = []
    for (ic, oc, k, _, _) in cfg.convs:
        lim = np.sqrt(6.0 / (ic * k * k + oc * k * k))
        params.append(rng.uniform(-lim, lim, oc * ic * k * k).astype(np.float32))
        params.append(np.zeros(oc, np.float32))
    F = cfg.flat_features()
    params.append(xavier(rng, F, cfg.classes))
    params.append(np.zeros(cfg.classes, np.float32))
    X = rng.uniform(0.0, 1.0, int(np.prod(cfg.input_shape))).astype(np.float32)
    labels = rng.integers(0, cfg.classes, cfg.batch)
    Y = np.zeros((cfg.classes, cfg.batch), np.float32)
    Y[labels, np.arange(cfg.batch)] = 1.0
    return params, X, Y.ravel()


@dataclass
class RNNConfig:
    """cell ("lstm" | "gru" | "rnn") over X [B, S, I] -> last hidden state -> Linear(H -> O) -> MSE."""
    name: str
    cell: str
    batch: int
    seq_len: int
    input_size: int
    hidden: int
    out_features: int = 1
    lr: float = 1e-3
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    seed: int = 1234
    loss: str = "mse"
    optimizer: str = "adam"
    opt_hyper: float = 0.9
    opt_eps: float = 1e-8


def rnn_config(config: int = 4, batch: int | None = None, seq_len: int | None = None,
               cell: str = "lstm") -> RNNConfig:
    """LSTM input 128, hidden 512, seq 64, batch 128,
    final hidden state -> Linear 512->1 -> MSE(mean)."""
    if config != 4:
        raise ValueError(f"config {config} is not the sequence config")
    return RNNConfig(f"C4 {cell.upper()} 128->512, T=64 -> 512->1, MSE", cell,
                     128 if batch is None else batch, 64 if seq_len is None else seq_len, 128, 512)


def synthetic_rnn(cfg: RNNConfig, rng: np.random.Generator):
    """W_ih, W_hh uniform with limits sqrt(6/(I+H)), sqrt(6/2H) (lstm.cpp:42-45);
    bias 0 with the LSTM forget block at 1 (lstm.cpp:47-49); Linear xavier;
    X ~ N(0,1) [B,S,I]; target ~ N(0,1) [B,1]."""
    G = GATES[cfg.cell] * cfg.hidden
    I, H = cfg.input_size, cfg.hidden
    lih, lhh = np.sqrt(6.0 / (I + H)), np.sqrt(6.0 / (2 * H))
    b = np.zeros(G, np.float32)
    if cfg.cell == "lstm":
        b[H:2 * H] = 1.0
    params = [rng.uniform(-lih, lih, I * G).astype(np.float32),
              rng.uniform(-lhh, lhh, H * G).astype(np.float32), b,
              xavier(rng, H, cfg.out_features), np.zeros(cfg.out_features, np.float32)]
    X = rng.standard_normal(cfg.batch * cfg.seq_len * I).astype(np.float32)
    Y = rng.standard_normal(cfg.batch * cfg.out_features).astype(np.float32)
    return params, X, Y


@dataclass
class TransformerConfig:
    """Embedding(vocab, D) -> blocks x [MHA(D, heads) + x -> BatchNorm(D) ->
    Linear(D -> ffn) -> GELU -> Linear(ffn -> D) + residual] -> MeanPool1D ->
    Linear(D -> classes) -> softmax-CE; token ids [B, S]."""
    name: str
    batch: int
    seq_len: int
    vocab: int
    embed_dim: int
    heads: int
    blocks: int
    ffn: int
    classes: int
    lr: float = 1e-3
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    seed: int = 1234
    loss: str = "softmax_ce"


def transformer_config(config: int = 5, batch: int | None = None, seq_len: int | None = None,
                       **shape) -> TransformerConfig:
    """vocab 8192, D 512, 8 heads, 2 blocks, FFN 2048,
    4 classes, B 32, S 256.  Keyword overrides shrink it for tests."""
    if config != 5:
        raise ValueError(f"config {config} is not the transformer config")
    c = TransformerConfig("C5 transformer Emb(8192,512) 2x[MHA(512,8)+res, BN, FFN 2048 GELU +res]"
                          " -> MeanPool1D -> 512->4", 32 if batch is None else batch,
                          256 if seq_len is None else seq_len, 8192, 512, 8, 2, 2048, 4)
    for k, v in shape.items():
        setattr(c, k, v)
    return c


def synthetic_transformer(cfg: TransformerConfig, rng: np.random.Generator):
    """Parameters in the session's order (embedding U(+-1/sqrt(D)) as
    embedding.cpp:38-39, MHA xavier as attention.cpp:47-50, gamma 1, beta 0,
    Linear xavier with zero bias), token ids uniform in [0, vocab) as int32
    ColMajor [B, S], one-hot uniform labels ColMajor [B, classes]."""
    D, F = cfg.embed_dim, cfg.ffn
    s = 1.0 / np.sqrt(D)
    params = [rng.uniform(-s, s, cfg.vocab * D).astype(np.float32)]
    for _ in range(cfg.blocks):
        params += [xavier(rng, D, D) for _ in range(4)]
        params += [np.ones(D, np.float32), np.zeros(D, np.float32)]
        params += [xavier(rng, D, F), np.zeros(F, np.float32), xavier(rng, F, D), np.zeros(D, np.float32)]
    params += [xavier(rng, D, cfg.classes), np.zeros(cfg.classes, np.float32)]
    ids = rng.integers(0, cfg.vocab, cfg.batch * cfg.seq_len).astype(np.int32)
    labels = rng.integers(0, cfg.classes, cfg.batch)
    Y = np.zeros((cfg.classes, cfg.batch), np.float32)
    Y[labels, np.arange(cfg.batch)] = 1.0
    return params, ids, Y.ravel()


@dataclass
class ResNetConfig:
    """The reference's residual benchmark network (residual_benckmark.cpp:104-152):
    Linear(in, W) -> ReLU -> depth x [Residual(Linear(W, W), Linear(W, w')) -> ReLU]
    -> Linear(w_last, classes) -> softmax-CE; w' = W except the last block's,
    which is last_width (a projection shortcut when it differs from W)."""
    name: str
    in_features: int
    width: int
    depth: int
    classes: int
    batch: int
    last_width: int = 0  # 0: width (identity shortcuts throughout)
    lr: float = 1e-3
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    seed: int = 1234
    loss: str = "softmax_ce"

    def __post_init__(self):
        if not self.last_width:
            self.last_width = self.width


def synthetic_resnet(cfg: ResNetConfig, rng: np.random.Generator):
    """Parameters in session order (he-uniform for the proj and block
    Linears as the benchmark builds them, init.cpp:49-61; xavier for the
    head and the projection, linear.hpp's default; biases 0), X ~ N(0,1)
    [B, in], one-hot uniform labels.  All ColMajor flat float32."""
    def he(i, o):
        lim = np.sqrt(6.0 / i)
        return rng.uniform(-lim, lim, i * o).astype(np.float32)
    W = cfg.width
    params = [he(cfg.in_features, W), np.zeros(W, np.float32)]
    for d in range(cfg.depth):
        w_out = cfg.last_width if d + 1 == cfg.depth else W
        params += [he(W, W), np.zeros(W, np.float32), he(W, w_out), np.zeros(w_out, np.float32)]
        if w_out != W:
            params.append(xavier(rng, W, w_out))
    w_last = cfg.last_width if cfg.depth else W
    params += [xavier(rng, w_last, cfg.classes), np.zeros(cfg.classes, np.float32)]
    X = rng.standard_normal(cfg.batch * cfg.in_features).astype(np.float32)
    labels = rng.integers(0, cfg.classes, cfg.batch)
    Y = np.zeros((cfg.classes, cfg.batch), np.float32)
    Y[labels, np.arange(cfg.batch)] = 1.0
    return params, X, Y.ravel()


def xavier(rng: np.random.Generator, fan_in: int, fan_out: int) -> np.ndarray:
    """xavier-uniform [fan_in, fan_out] (init.cpp:21-33), ColMajor flat."""
    lim = np.sqrt(6.0 / (fan_in + fan_out))
    return rng.uniform(-lim, lim, fan_in * fan_out).astype(np.float32)


def synthetic_mlp(cfg: MLPConfig, rng: np.random.Generator):
    """Parameters (W, b per layer; b = 0 as linear.cpp:75-80), X ~ N(0,1) and
    targets (Bernoulli(0.5) for BCE, one-hot uniform labels for softmax-CE and
    categorical CE, N(0,1) for MSE / MAE / Huber), all ColMajor flat float32."""
    params = []
    for i, o in zip(cfg.sizes[:-1], cfg.sizes[1:]):
        params.append(xavier(rng, i, o))
        params.append(np.zeros(o, np.float32))
    B, I, O = cfg.batch, cfg.sizes[0], cfg.sizes[-1]
    X = rng.standard_normal(B * I).astype(np.float32)
    if cfg.loss == "bce":
        Y = (rng.uniform(size=B * O) < 0.5).astype(np.float32)
    elif cfg.loss in ("softmax_ce", "cce"):
        labels = rng.integers(0, O, B)
        Y = np.zeros((O, B), np.float32)
        Y[labels, np.arange(B)] = 1.0
        Y = Y.ravel()  # ColMajor [B, O]: column o = class o
    else:
        Y = rng.standard_normal(B * O).astype(np.float32)
    return params, X, Y


def _onehot(rng, B, C):
    labels = rng.integers(0, C, B)
    Y = np.zeros((C, B), np.float32)
    Y[labels, np.arange(B)] = 1.0
    return Y.ravel()


def synthetic_batch(cfg, rng: np.random.Generator):
    """A fresh (X, Y) batch of a config, from the same distributions as its
    synthetic_* generator, without drawing parameters (long runs take a new
    batch every step)."""
    if isinstance(cfg, MLPConfig):
        B, I, O = cfg.batch, cfg.sizes[0], cfg.sizes[-1]
        X = rng.standard_normal(B * I).astype(np.float32)
        if cfg.loss == "bce":
            return X, (rng.uniform(size=B * O) < 0.5).astype(np.float32)
        if cfg.loss in ("softmax_ce", "cce"):
            return X, _onehot(rng, B, O)
        return X, rng.standard_normal(B * O).astype(np.float32)
    if isinstance(cfg, CNNConfig):
        X = rng.uniform(0.0, 1.0, int(np.prod(cfg.input_shape))).astype(np.float32)
        return X, _onehot(rng, cfg.batch, cfg.classes)
    if isinstance(cfg, RNNConfig):
        X = rng.standard_normal(cfg.batch * cfg.seq_len * cfg.input_size).astype(np.float32)
        return X, rng.standard_normal(cfg.batch * cfg.out_features).astype(np.float32)
    if isinstance(cfg, TransformerConfig):
        ids = rng.integers(0, cfg.vocab, cfg.batch * cfg.seq_len).astype(np.int32)
        return ids, _onehot(rng, cfg.batch, cfg.classes)
    if isinstance(cfg, ResNetConfig):
        X = rng.standard_normal(cfg.batch * cfg.in_features).astype(np.float32)
        return X, _onehot(rng, cfg.batch, cfg.classes)
    raise TypeError(f"no batch generator for {type(cfg).__name__}")


class Session:
    """One C++ training session (model + loss + Adam + stream) on cuda:0."""

    def __init__(self, cfg):
        lib = load()
        h = C.c_void_p()
        self.tokens = isinstance(cfg, TransformerConfig)
        if self.tokens:
            _check(lib.cnt_transformer_create(C.byref(h), cfg.batch, cfg.seq_len, cfg.vocab,
                                              cfg.embed_dim, cfg.heads, cfg.blocks, cfg.ffn,
                                              cfg.classes, cfg.lr, cfg.beta1, cfg.beta2, cfg.eps,
                                              cfg.seed))
            self.x_size = cfg.batch * cfg.seq_len
            self.y_size = cfg.batch * cfg.classes
        elif isinstance(cfg, ResNetConfig):
            _check(lib.cnt_resnet_create(C.byref(h), cfg.in_features, cfg.width, cfg.depth, cfg.last_width,
                                         cfg.classes, cfg.batch, cfg.lr, cfg.beta1, cfg.beta2, cfg.eps,
                                         cfg.seed))
            self.x_size = cfg.batch * cfg.in_features
            self.y_size = cfg.batch * cfg.classes
        elif isinstance(cfg, RNNConfig):
            _check(lib.cnt_rnn_create(C.byref(h), CELL[cfg.cell], cfg.batch,
                                      cfg.seq_len, cfg.input_size, cfg.hidden, cfg.out_features,
                                      cfg.lr, cfg.beta1, cfg.beta2, cfg.eps, cfg.seed))
            self.x_size = cfg.batch * cfg.seq_len * cfg.input_size
            self.y_size = cfg.batch * cfg.out_features
        elif isinstance(cfg, CNNConfig):
            spec = [v for c in cfg.convs for v in c]
            _check(lib.cnt_cnn_create(C.byref(h), len(cfg.convs), (C.c_int64 * len(spec))(*spec),
                                      cfg.pool, (C.c_int64 * 4)(*cfg.input_shape), cfg.classes,
                                      cfg.lr, cfg.beta1, cfg.beta2, cfg.eps, cfg.seed))
            self.x_size = int(np.prod(cfg.input_shape))
            self.y_size = cfg.batch * cfg.classes
        else:
            sizes = (C.c_int64 * len(cfg.sizes))(*cfg.sizes)
            _check(lib.cnt_mlp_create_ex(C.byref(h), len(cfg.sizes) - 1, sizes, ACT[cfg.hidden_act],
                                         ACT[cfg.out_act], LOSS[cfg.loss], cfg.batch, cfg.lr,
                                         cfg.beta1, cfg.beta2, cfg.eps, cfg.seed, cfg.dropout))
            self.x_size = cfg.batch * cfg.sizes[0]
            self.y_size = cfg.batch * cfg.sizes[-1]
        self.h = h
        self.cfg = cfg
        opt = getattr(cfg, "optimizer", "adam")
        if opt != "adam":
            _check(lib.cnt_set_optimizer(h, OPT[opt], cfg.opt_hyper, cfg.opt_eps))

    def close(self):
        if self.h:
            _check(load().cnt_destroy(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return load().cnt_stream(self.h) or 0

    def num_params(self) -> int:
        n = C.c_int()
        _check(load().cnt_num_params(self.h, C.byref(n)))
        return n.value

    def param_size(self, i: int) -> int:
        n = C.c_int64()
        _check(load().cnt_param_size(self.h, i, C.byref(n)))
        return n.value

    def set_params(self, params) -> None:
        assert len(params) == self.num_params()
        for i, p in enumerate(params):
            p = np.ascontiguousarray(p, np.float32)
            assert p.size == self.param_size(i), f"param {i}: size {p.size} != {self.param_size(i)}"
            _check(load().cnt_set_param(self.h, i, p.ctypes.data))

    def get_params(self) -> list:
        out = []
        for i in range(self.num_params()):
            a = np.empty(self.param_size(i), np.float32)
            _check(load().cnt_get_param(self.h, i, a.ctypes.data))
            out.append(a)
        return out

    def get_grads(self) -> list:
        out = []
        for i in range(self.num_params()):
            a = np.empty(self.param_size(i), np.float32)
            _check(load().cnt_get_grad(self.h, i, a.ctypes.data))
            out.append(a)
        return out

    def get_opt_state(self, k: int) -> tuple[list, list]:
        """The optimizer's state tensor k of every parameter (Adam: 0 m, 1 v)
        in get_params' layout, and each parameter's step count t."""
        out, ts = [], []
        for i in range(self.num_params()):
            a = np.empty(self.param_size(i), np.float32)
            t = C.c_int()
            _check(load().cnt_get_opt_state(self.h, i, k, a.ctypes.data, C.byref(t)))
            out.append(a)
            ts.append(t.value)
        return out, ts

    def set_batch(self, X: np.ndarray, Y: np.ndarray) -> None:
        """X: float32 inputs, or int32 token ids for a transformer session."""
        X = np.ascontiguousarray(X, np.int32 if self.tokens else np.float32)
        Y = np.ascontiguousarray(Y, np.float32)
        assert X.size == self.x_size, f"X has {X.size} values, the model takes {self.x_size}"
        assert Y.size == self.y_size, f"Y has {Y.size} values, the model takes {self.y_size}"
        fn = load().cnt_set_batch_tokens if self.tokens else load().cnt_set_batch
        _check(fn(self.h, X.ctypes.data, Y.ctypes.data))

    def set_batch_device(self, X_ptr: int, Y_ptr: int) -> None:
        _check(load().cnt_set_batch_device(self.h, X_ptr, Y_ptr))

    def step(self, read_loss: bool = True) -> float | None:
        if read_loss:
            loss = C.c_float()
            _check(load().cnt_step(self.h, C.byref(loss)))
            return loss.value
        _check(load().cnt_step(self.h, None))
        return None

    def forward_backward(self) -> float:
        """zero_grad, forward, loss, backward; returns the loss (grads readable)."""
        loss = C.c_float()
        _check(load().cnt_forward_backward(self.h, C.byref(loss)))
        return loss.value

    def update(self) -> None:
        _check(load().cnt_update(self.h))

    def save_model(self, path) -> None:
        """The reference's CNET model file (weights of Linear / BatchNorm / Embedding)."""
        _check(load().cnt_save_model(self.h, str(path).encode()))

    def load_model(self, path) -> None:
        _check(load().cnt_load_model(self.h, str(path).encode()))

    def save_checkpoint(self, path) -> None:
        """CNET records + every parameter and the optimizer state (exact resume)."""
        _check(load().cnt_save_checkpoint(self.h, str(path).encode()))

    def load_checkpoint(self, path) -> None:
        _check(load().cnt_load_checkpoint(self.h, str(path).encode()))

    def synchronize(self) -> None:
        _check(load().cnt_synchronize(self.h))

    def set_fused_step(self, enable: bool) -> None:
        """Whether steps may run the fused two-launch step of the MLP
        benchmark model (default on; cnt_set_fused_step)."""
        _check(load().cnt_set_fused_step(self.h, int(enable)))

    def capture(self) -> None:
        """Records zero_grad + forward + loss + backward into a HIP graph that
        later step() calls replay (Adam runs eagerly after each replay).  Needs
        one eager step first."""
        _check(load().cnt_capture_step(self.h))

    def release_graph(self) -> None:
        _check(load().cnt_release_graph(self.h))

    @property
    def has_graph(self) -> bool:
        return bool(load().cnt_has_graph(self.h))


def npy_save(path, colmajor: np.ndarray, dims) -> None:
    """Writes float32 ColMajor data of shape dims as .npy (fortran_order True)."""
    a = np.ascontiguousarray(colmajor, np.float32).ravel()
    d = (C.c_int64 * len(dims))(*dims)
    _check(load().cnt_npy_save(str(path).encode(), a.ctypes.data, len(dims), d))


def npy_load(path, raw_colmajor: bool = False):
    """Reads a float32 .npy file; returns (ColMajor flat data, dims)."""
    import os
    cap = max(os.path.getsize(path) // 4, 1)
    out = np.empty(cap, np.float32)
    nd = C.c_int(16)
    dims = (C.c_int64 * 16)()
    _check(load().cnt_npy_load(str(path).encode(), out.ctypes.data, cap, C.byref(nd), dims,
                               1 if raw_colmajor else 0))
    d = [int(dims[i]) for i in range(nd.value)]
    return out[:int(np.prod(d))].copy(), d


STAGE = {"resident": 1, "stream": 2}


class Loader:
    """Utils::DataLoader through the C ABI: features [N, F] and labels [N, L]
    as ColMajor flat float32 (Eigen's order)."""

    def __init__(self, features, labels, n, f, l, batch, shuffle=True, drop_last=False, seed=0):
        lib = load()
        self._x = np.ascontiguousarray(features, np.float32).ravel()
        self._y = np.ascontiguousarray(labels, np.float32).ravel()
        assert self._x.size == n * f and self._y.size == n * l
        h = C.c_void_p()
        _check(lib.cnt_loader_create(C.byref(h), self._x.ctypes.data, self._y.ctypes.data, n, f, l, batch,
                                     int(shuffle), int(drop_last), seed))
        self.h, self.n, self.f, self.l, self.batch = h, n, f, l, batch

    def close(self):
        if self.h:
            _check(load().cnt_loader_destroy(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def num_batches(self) -> int:
        c = C.c_int64()
        _check(load().cnt_loader_num_batches(self.h, C.byref(c)))
        return c.value

    def indices(self) -> np.ndarray:
        out = np.empty(self.n, np.int32)
        _check(load().cnt_loader_indices(self.h, out.ctypes.data))
        return out

    def reset(self) -> None:
        _check(load().cnt_loader_reset(self.h))

    def host_batch(self, k: int):
        x = np.empty(self.batch * self.f, np.float32)
        y = np.empty(self.batch * self.l, np.float32)
        bs = C.c_int64()
        _check(load().cnt_loader_host_batch(self.h, k, x.ctypes.data, y.ctypes.data, C.byref(bs)))
        return x[:bs.value * self.f].copy(), y[:bs.value * self.l].copy(), bs.value

    def to_device(self, mode: str) -> None:
        _check(load().cnt_loader_to_device(self.h, STAGE[mode]))

    def next(self, x_ptr: int, y_ptr: int, stream: int = 0) -> int:
        """The epoch's next batch into device buffers; returns its size (0 at the end)."""
        bs = C.c_int64()
        _check(load().cnt_loader_next(self.h, x_ptr, y_ptr, C.byref(bs), stream))
        return bs.value

    def next_batch(self, sess: "Session") -> int:
        bs = C.c_int64()
        _check(load().cnt_loader_next_batch(self.h, sess.h, C.byref(bs)))
        return bs.value
