"""Benchmark: fp32 train step (forward + backward + Adam) of a BASELINE config
on one MI355X.  The default is config 2, the workload the metric is quoted
on: the wide MLP classifier Linear 1024->4096 -> ReLU -> Linear 4096->4096
-> ReLU -> Linear 4096->10, softmax cross-entropy (mean), Adam(1e-3, 0.9,
0.999, 1e-8), batch 4096.  --config 1|3|4|5 measures the other configs the
same way (MLP 30-64-1; CNN; LSTM 128->512 T=64; transformer encoder).

The step runs in the C++ trainer (libcppnet.so: CppNet-compatible classes on
device "gpu") on its own HIP stream; inputs, weights, gradients and Adam
moments are resident in HBM before timing starts.  Prints ONE JSON line:

  value            train samples/s = batch * steps / timed seconds
  roofline         the dominant kernel class, the fp32 MFMA GEMM-shaped kernels
                   (the GEMM kernel; for config 3 also the implicit-GEMM conv
                   kernels): algorithmic flops per launch / average launch
                   duration, measured live with HIP events on the launch
                   stream around every such launch of a few extra steps
  hbm_kernels      each bandwidth-bound kernel of the step: algorithmic bytes per
                   launch / event-timed launch duration, against 8 TB/s
  cpu_baseline     the CPU oracle (a restatement of the reference's cpu-eigen
                   semantics, oracle/) on a bounded sample of the same workload
  other_configs    the four other configs, GPU legs only, timed the same way
                   (20 steps each, config 1: 200): samples/s, ms/step, their
                   roofline and their four longest bandwidth-bound kernels;
                   --only leaves them out

Usage: python bench.py [--gpus 1] [--config 2] [--steps K] [--warmup W]
                       [--no-cpu-baseline] [--cpu-seconds S] [--graph] [--only]

--graph replays the step's zero_grad + forward + loss + backward as one
captured HIP graph (cnt_capture_step) and then runs the fused Adam update
eagerly; the default launches every kernel from the host.  Both compute the
same step, bit for bit.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "train samples/sec (fwd+bwd+Adam, fp32) + backward % of fp32/HBM roofline"
PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense fp32 matrix
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- workloads
# Step flops = forward + weight gradients + input gradients (3x the forward
# products), less the first layer's input gradient: the train step does not
# compute it (its input is data), so it is not counted as work done.
def _mlp_flops(cfg):
    per_layer = [2.0 * cfg.batch * i * o for i, o in zip(cfg.sizes[:-1], cfg.sizes[1:])]
    return 3 * sum(per_layer) - per_layer[0]


def _cnn_flops(cfg):
    N, C, H, W = cfg.input_shape
    fwd, first = 0.0, None
    for (ic, oc, k, s, p) in cfg.convs:
        HO, WO = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
        f = 2.0 * N * HO * WO * oc * ic * k * k
        first = f if first is None else first
        fwd += f
        H, W = (HO - cfg.pool) // cfg.pool + 1, (WO - cfg.pool) // cfg.pool + 1
    fwd += 2.0 * N * cfg.flat_features() * cfg.classes
    return 3 * fwd - first


def _rnn_flops(cfg):
    G = (4 if cfg.cell == "lstm" else 3) * cfg.hidden
    x_proj = 2.0 * cfg.batch * cfg.seq_len * cfg.input_size * G
    fwd = x_proj + 2.0 * cfg.batch * cfg.seq_len * cfg.hidden * G
    fwd += 2.0 * cfg.batch * cfg.hidden * cfg.out_features
    return 3 * fwd - x_proj


def _tr_flops(cfg):
    BS, D, S = cfg.batch * cfg.seq_len, cfg.embed_dim, cfg.seq_len
    blk = 4 * 2.0 * BS * D * D + 2 * 2.0 * cfg.batch * S * S * D + 2 * 2.0 * BS * D * cfg.ffn
    return 3 * (cfg.blocks * blk + 2.0 * cfg.batch * D * cfg.classes)


def workload(config: int, batch: int | None = None):
    """(cfg, synthetic-data function, oracle class, flops function, description)"""
    from cppnet_amd import trainer
    if config in (1, 2):
        from oracle.mlp import OracleMLP
        cfg = trainer.mlp_config(config, batch=batch)
        desc = {1: "config 1: MLP 30-64-1, sigmoid, BCE, Adam",
                2: "config 2: wide MLP 1024-4096-4096-10, softmax-CE, Adam"}[config]
        return cfg, trainer.synthetic_mlp, OracleMLP, _mlp_flops, desc
    if config == 3:
        from oracle.cnn import OracleCNN
        cfg = trainer.cnn_config(3, batch=batch)
        return (cfg, trainer.synthetic_cnn, OracleCNN, _cnn_flops,
                "config 3: CNN 2x(conv3x3, ReLU, maxpool2) -> 4096->10, softmax-CE, Adam")
    if config == 4:
        from oracle.rnn import OracleSeqRegressor
        cfg = trainer.rnn_config(4, batch=batch)
        return (cfg, trainer.synthetic_rnn, OracleSeqRegressor, _rnn_flops,
                "config 4: LSTM 128->512, T=64, last hidden -> 512->1, MSE, Adam")
    if config == 5:
        from oracle.transformer import OracleTransformer
        cfg = trainer.transformer_config(5, batch=batch)
        return (cfg, trainer.synthetic_transformer, OracleTransformer, _tr_flops,
                "config 5: transformer Emb(8192,512) -> 2x[MHA(512,8)+res, BatchNorm, "
                "512-2048 GELU 2048-512 +res] -> MeanPool1D -> 512->4, softmax-CE, Adam")
    raise ValueError(f"unknown config {config}")


CPU_BATCH = {1: 512, 2: 512, 3: 32, 4: 16, 5: 4}
# Batch of the reference's "cpu" device leg (Linear as OpenMP loops over the
# outputs, linear.cpp:196-330) for the MLP configs: those loops walk the
# ColMajor inputs with a stride of the batch, ~40x slower than the contraction
# at C2's widths, so C2's leg runs 64 samples a step.
CPU_LOOPS_BATCH = {1: 512, 2: 64}

# HBM bytes per launch of each config's dominant kernel class, from the two
# rocprofv3 PMC runs (FETCH_SIZE, WRITE_SIZE) of that config scaled by a
# reference kernel of known traffic (bench.py --traffic-calibration),
# averaged over the class's launches of a step; the runs, the factors and the
# per-kernel tables are in profiles/*_counters.md.
PMC_TRAFFIC_BYTES = {1: 0.6e6, 2: 471.9e6, 3: 39.3e6, 4: 955.1e6, 5: 170.4e6}


def _cpu_model() -> str:
    """The host's "model name" from /proc/cpuinfo with its family, model and
    stepping numbers (some hosts report only a family name such as "AMD EPYC")."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" in line:
                    k, v = (x.strip() for x in line.split(":", 1))
                    info.setdefault(k, v)
                if not line.strip() and info:
                    break
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    ids = [f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info]
    return f"{name} ({', '.join(ids)})" if ids else name


def _cpu_share() -> int:
    """Host threads this process may use: its affinity set, capped at the 16
    host cores one GPU's share of the box holds."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _time_oracle(o, config: int, batch: int, threads: int, seconds_budget: float, max_steps: int):
    import numpy as np
    o.cnref_set_threads(threads)
    cfg, synth, Oracle, _, _ = workload(config, batch=batch)
    params, X, Y = synth(cfg, np.random.default_rng(99))
    ref = Oracle(cfg, o)
    ref.keep = False
    ref.set_params(params)
    ref.step(X, Y)  # warm-up
    n, t0 = 0, time.perf_counter()
    while True:
        ref.step(X, Y)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds_budget or n >= max_steps:
            break
    return {"threads": threads, "batch": batch, "steps": n, "seconds": round(el, 2),
            "samples_per_s": round(batch * n / el, 2)}


def cpu_baseline(config: int, seconds_budget: float = 20.0):
    """Times the oracle-composed model (oracle/ over oracle/liboracle.so, a
    plain C++ restatement of the reference's cpu-eigen semantics) on this
    host: the same step at a reduced batch on all the host threads of this
    GPU's share (the reported value) and on 4 threads, each for about
    seconds_budget / 2 of CPU work after a warm-up step; for config 2 also one
    step at the full batch.  Figures are samples/s."""
    from oracle import load_oracle

    o = load_oracle()
    share = _cpu_share()
    batch = CPU_BATCH[config]
    max_steps = 20000 if config == 1 else 50
    eigen = lambda **kw: dict(device="cpu-eigen", **kw)
    legs = [eigen(**_time_oracle(o, config, batch, share, seconds_budget / 2, max_steps))]
    if share != 4:
        legs.append(eigen(**_time_oracle(o, config, batch, 4, seconds_budget / 2, max_steps)))
    # one thread: the reference's cpu-eigen contractions run on the calling
    # thread (no Eigen ThreadPoolDevice) and its Conv2D backward is a serial
    # loop, so this leg is the closer figure for that device
    legs.append(eigen(**_time_oracle(o, config, batch, 1, seconds_budget / 4, max_steps)))
    full = workload(config)[0].batch
    if config == 2:
        legs.append(eigen(**_time_oracle(o, config, full, share, 0.0, 1)))
    if config in CPU_LOOPS_BATCH:
        # the reference's "cpu" device: the same step with Linear as its OpenMP loops
        o.cnref_set_cpu_loops(1)
        try:
            for threads in dict.fromkeys((share, 4)):
                legs.append(dict(device="cpu", **_time_oracle(o, config, CPU_LOOPS_BATCH[config], threads,
                                                              seconds_budget / 4, max_steps)))
        finally:
            o.cnref_set_cpu_loops(0)
    main = legs[0]
    return {"value": main["samples_per_s"], "unit": "samples/s", "cores": share,
            "kind": "port", "cpu_model": _cpu_model(),
            "legs": legs,
            "sample": (f"reference-semantics restatement (oracle/, plain C++ of the cpu-eigen "
                       f"semantics, OpenMP): {main['steps']} train steps of config {config} at batch "
                       f"{batch} (of {full}) on {share} threads in {main['seconds']} s; legs also "
                       f"time 4 threads, 1 thread" + (" and one full-batch step" if config == 2 else "") +
                       (f", and the reference's \"cpu\" device (Linear as OpenMP loops over the outputs) "
                        f"at batch {CPU_LOOPS_BATCH[config]} on {share} and 4 threads"
                        if config in CPU_LOOPS_BATCH else ""))}


def traffic_calibration() -> int:
    """A kernel whose HBM traffic is known, for scaling PMC byte counters:
    cnhip_add(a, b, c, n) reads 2n floats and writes n."""
    import ctypes as C
    from cppnet_amd import _capi
    lib = _capi.load()
    n = 64 * 1024 * 1024
    bufs = [C.c_void_p() for _ in range(3)]
    for q in bufs:
        _capi.check(lib.cnhip_malloc(C.byref(q), n * 4))
        _capi.check(lib.cnhip_memset_async(q, 0, n * 4, None))
    for _ in range(5):
        _capi.check(lib.cnhip_add(bufs[0], bufs[1], bufs[2], n, None))
    _capi.check(lib.cnhip_device_synchronize())
    for q in bufs:
        _capi.check(lib.cnhip_free(q))
    log(f"bench.py: traffic calibration done (cnhip_add, n = {n}, 5 launches)")
    return 0


PHASES = {"forward": ["wait for h_{t-1} (first poll sent, x_{t+1} staged)", "stage h_{t-1} and the block's vote",
                     "recurrent product (MFMA), gates", "cell update, h_t handed on, caches written"],
          "backward": ["weight-gradient MFMAs of step t+1", "wait for the partials of step t+1",
                       "their sum and the block's vote", "cell backward, dG_t staged",
                       "recurrent partials dG_t W_hh^T (MFMA) handed on"]}


def phase_stamps(config: int = 4) -> int:
    """Per-phase time of the persistent LSTM kernels' timesteps: one train
    step of the config with cnhip_lstm_phase_stamps set, then the mean over
    blocks and the interior timesteps of each phase's span (the kernels
    record a 100 MHz realtime counter at every phase boundary)."""
    import ctypes as C

    import numpy as np
    import torch
    from cppnet_amd import _capi, trainer

    lib = _capi.load()
    cfg, synth, _, _, desc = workload(config)
    params, X, Y = synth(cfg, np.random.default_rng(2024))
    sess = trainer.Session(cfg)
    sess.set_params(params)
    sess.set_batch(X, Y)
    for _ in range(3):
        sess.step(read_loss=False)
    sess.synchronize()
    S, blocks = cfg.seq_len, (cfg.batch // 16) * (cfg.hidden // 16)
    cap = blocks * S * 8
    bufs = [torch.zeros(cap, dtype=torch.int64, device="cuda") for _ in range(2)]
    torch.cuda.synchronize()
    _capi.check(lib.cnhip_lstm_phase_stamps(C.c_void_p(bufs[0].data_ptr()), C.c_void_p(bufs[1].data_ptr()), cap))
    try:
        sess.step(read_loss=False)
        sess.synchronize()
    finally:
        _capi.check(lib.cnhip_lstm_phase_stamps(None, None, 0))
    out = {"workload": desc, "clock_MHz": 100, "timesteps": S, "blocks": blocks}
    for k, (name, b) in enumerate(zip(("forward", "backward"), bufs)):
        st = b.cpu().numpy().reshape(blocks, S, 8).astype(np.float64)
        n = len(PHASES[name])
        if name == "forward":  # steps 1 .. S-2, phases 0 .. n in time order
            sl = st[:, 1:S - 1, :n + 1]
        else:  # steps S-2 .. 1 (t descending in time)
            sl = st[:, 1:S - 1, :n + 1]
        d = np.diff(sl, axis=2) / 100.0  # us
        step_us = (sl[:, :, n] - sl[:, :, 0]) / 100.0
        if name == "forward":
            nxt = (st[:, 2:S, 0] - st[:, 1:S - 1, 0]) / 100.0
        else:
            nxt = (st[:, 0:S - 2, 0] - st[:, 1:S - 1, 0]) / 100.0
        out[name] = {"phases_us": {PHASES[name][i]: round(float(d[:, :, i].mean()), 3) for i in range(n)},
                     "step_us": round(float(nxt.mean()), 3),
                     "step_us_max_over_blocks": round(float(nxt.mean(axis=1).max()), 3),
                     "span_us": round(float((st[:, :, 0].max() - st[:, :, 0].min()) / 100.0), 1)}
        log(f"bench.py: {name}: " + ", ".join(f"{k2} {v:.2f} us" for k2, v in out[name]["phases_us"].items()) +
            f"; step {out[name]['step_us']:.2f} us")
    sess.close()
    print(json.dumps({"phase_stamps": out}))
    return 0


SMALL_CLASS = {
    "mlp2_bce_part_kernel": "mlp2_bce_part_kernel (the fused step's forward, loss and backward with per-block "
                            "gradient sums; the step is launch-latency bound)",
    "gemm_small_kernel": "gemm_small_thread/wave_kernel (SIMT fp32 GEMMs of <= 2 MFLOP: the "
                         "step is launch-latency bound)"}


def small_roofline(hbm_kernels, step_ms, config):
    """A step without MFMA launches (config 1: the fused two-launch step, or
    with it switched off, latency-bound SIMT GEMMs): the dominant kernel against
    HBM, its algorithmic bytes over its event-timed launch duration."""
    k = next((r for name in SMALL_CLASS for r in hbm_kernels if r["kernel"] == name), None)
    if k is None:
        return None
    return {"bound": "hbm", "kernel": SMALL_CLASS[k["kernel"]],
            "achieved": k["achieved_GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": k["frac"],
            "traffic": PMC_TRAFFIC_BYTES.get(config), "traffic_unit": "bytes per launch (rocprofv3 PMC, see profiles/)",
            "launches_per_step": k["launches_per_step"], "avg_launch_us": k["avg_us"],
            "bytes_per_launch": k["bytes_per_launch"],
            "share_of_step": round(k["avg_us"] * k["launches_per_step"] / (step_ms * 1e3), 3)}


def loader_leg(sess, cfg, B, steps, step_ms, mode):
    """`steps` train steps whose batches come from a DataLoader over a synthetic
    dataset of 16 batches (reshuffled at each epoch's end, inside the timed
    region), with the step's inputs delivered by cnt_loader_next_batch."""
    import ctypes as C

    import numpy as np
    from cppnet_amd import _capi, trainer

    lib = _capi.load()
    nb = 16
    F = sess.x_size // B
    L = sess.y_size // B
    N = nb * B
    rng = np.random.default_rng(7)
    Xd = rng.standard_normal(N * F, dtype=np.float32)
    Yd = np.zeros((N, L), np.float32)
    Yd[np.arange(N), rng.integers(0, L, N)] = 1.0  # one-hot rows (valid for every loss here)
    ld = trainer.Loader(Xd, Yd.ravel(order="F"), N, F, L, B, True, True, seed=3)
    ld.to_device(mode)

    def feed():
        if ld.next_batch(sess) == 0:
            ld.reset()
            ld.next_batch(sess)

    for _ in range(3):
        feed()
        sess.step(read_loss=False)
    sess.synchronize()
    ev0, ev1 = C.c_void_p(), C.c_void_p()
    _capi.check(lib.cnhip_event_create(C.byref(ev0)))
    _capi.check(lib.cnhip_event_create(C.byref(ev1)))
    t0 = time.perf_counter()
    _capi.check(lib.cnhip_event_record(ev0, sess.stream))
    for _ in range(steps):
        feed()
        sess.step(read_loss=False)
    _capi.check(lib.cnhip_event_record(ev1, sess.stream))
    sess.synchronize()
    wall = time.perf_counter() - t0
    ms = C.c_float()
    _capi.check(lib.cnhip_event_elapsed_ms(C.byref(ms), ev0, ev1))
    per = max(ms.value, wall * 1e3) / steps  # the host side can be the longer clock
    gather = None
    if mode == "resident":  # the batch-assembly kernel's own HBM rate, event-timed
        _capi.check(lib.cnhip_hbm_timing_enable(1))
        for _ in range(5):
            feed()
            sess.step(read_loss=False)
        rows = [r for r in _capi.hbm_timing_rows() if r["kernel"] == "gather_rows_kernel"]
        _capi.check(lib.cnhip_hbm_timing_enable(0))
        if rows and rows[0]["total_ms"] > 0:
            r = rows[0]
            gbs = r["total_bytes"] / (r["total_ms"] * 1e-3) / 1e9
            gather = {"kernel": "gather_rows_kernel", "avg_us": round(r["total_ms"] * 1e3 / r["launches"], 2),
                      "bytes_per_launch": round(r["total_bytes"] / r["launches"]),
                      "achieved_GBs": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}
    ld.close()
    out = {"mode": mode, "samples_per_s": round(B / (per * 1e-3), 1), "ms_per_step": round(per, 4),
           "vs_resident_inputs": round(step_ms / per, 3), "dataset_batches": nb,
           "bytes_per_batch": B * (F + L) * 4}
    if gather:
        out["gather_kernel"] = gather
    if mode == "stream":
        out["host_to_device_GBs_needed"] = round(B * (F + L) * 4 / (per * 1e-3) / 1e9, 2)
    log(f"bench.py: loader {mode}: {per:.4f} ms/step ({out['vs_resident_inputs']:.3f} of resident inputs)")
    return out


KERNEL_CLASS = {
    3: "gemm_f32_kernel + conv_pixel/conv_wgrad/conv_wgrad_px_kernel (fp32 MFMA, all shapes of the step)",
    4: "gemm_f32_kernel + lstm_fwd/bwd_persist_kernel (fp32 MFMA; the whole recurrence of "
       "each pass in one launch, cell update fused, the backward also accumulating "
       "dW_hh, dW_ih and db)"}
DEFAULT_KERNEL_CLASS = "gemm_f32_kernel (fp32 MFMA GEMM, all shapes of the step; gemm_pair_kernel where two run in one launch)"


def measure(config: int, steps: int, warmup: int, graph: bool = False, loader: str | None = None,
            hbm_detail: bool = True, fused: bool = True) -> dict:
    """Times `steps` train steps of one config after `warmup` untimed ones,
    inputs resident in HBM, between HIP events on the session's stream; then
    three more eager steps with per-launch events around the MFMA class and
    three around the bandwidth-bound kernels.  Returns the per-config part of
    the JSON line (no cpu_baseline)."""
    import ctypes as C

    import numpy as np
    from cppnet_amd import _capi, trainer

    lib = _capi.load()
    cfg, synth, _, flops_fn, desc = workload(config)
    B = cfg.batch
    params, X, Y = synth(cfg, np.random.default_rng(2024))
    sess = trainer.Session(cfg)
    sess.set_fused_step(fused)
    sess.set_params(params)
    sess.set_batch(X, Y)           # resident in HBM from here on
    stream = sess.stream
    log(f"bench.py: {desc}, batch {B}: {warmup} warmup + {steps} timed steps")

    for _ in range(warmup):
        sess.step(read_loss=False)
    if graph:
        # zero_grad + forward + loss + backward replayed as one HIP graph; the
        # Adam update still runs every step, eagerly, after the replay
        sess.capture()
        for _ in range(2):
            sess.step(read_loss=False)
    sess.synchronize()

    ev0, ev1 = C.c_void_p(), C.c_void_p()
    _capi.check(lib.cnhip_event_create(C.byref(ev0)))
    _capi.check(lib.cnhip_event_create(C.byref(ev1)))
    t0 = time.perf_counter()
    _capi.check(lib.cnhip_event_record(ev0, stream))
    for _ in range(steps):
        sess.step(read_loss=False)
    _capi.check(lib.cnhip_event_record(ev1, stream))
    sess.synchronize()
    wall = time.perf_counter() - t0
    ms = C.c_float()
    _capi.check(lib.cnhip_event_elapsed_ms(C.byref(ms), ev0, ev1))
    _capi.check(lib.cnhip_event_destroy(ev0))
    _capi.check(lib.cnhip_event_destroy(ev1))
    step_ms = ms.value / steps
    loss = sess.step()  # one more step, read back: the run trained on finite numbers
    if not np.isfinite(loss):
        sess.close()
        raise RuntimeError(f"config {config}: non-finite loss {loss}")
    log(f"bench.py: config {config}: {step_ms:.4f} ms/step, loss {loss:.6f}")

    # Dominant kernel class: per-launch timing over a few extra eager steps
    # (a graph replay records no per-launch events).
    if sess.has_graph:
        sess.release_graph()
    prof_steps = 3
    _capi.check(lib.cnhip_gemm_timing_enable(1))
    for _ in range(prof_steps):
        sess.step(read_loss=False)
    launches, kms, kfl = C.c_int64(), C.c_double(), C.c_double()
    _capi.check(lib.cnhip_gemm_timing_read(C.byref(launches), C.byref(kms), C.byref(kfl)))
    _capi.check(lib.cnhip_gemm_timing_enable(0))
    per_launch_us = kms.value * 1e3 / max(1, launches.value)
    flops_per_launch = kfl.value / max(1, launches.value)
    achieved = kfl.value / (kms.value * 1e-3) / 1e12 if kms.value > 0 else 0.0  # TFLOP/s
    gemm_share = kms.value / prof_steps / step_ms

    # Bandwidth-bound kernels: per-launch timing over a few more eager steps,
    # each launch credited with its algorithmic HBM bytes.
    _capi.check(lib.cnhip_hbm_timing_enable(1))
    for _ in range(prof_steps):
        sess.step(read_loss=False)
    hbm_rows = _capi.hbm_timing_rows()
    _capi.check(lib.cnhip_hbm_timing_enable(0))
    hbm_kernels = []
    for r in sorted(hbm_rows, key=lambda r: -r["total_ms"]):
        gbs = r["total_bytes"] / (r["total_ms"] * 1e-3) / 1e9 if r["total_ms"] > 0 else 0.0
        hbm_kernels.append({"kernel": r["kernel"],
                            "launches_per_step": round(r["launches"] / prof_steps, 2),
                            "avg_us": round(r["total_ms"] * 1e3 / r["launches"], 2),
                            "bytes_per_launch": round(r["total_bytes"] / r["launches"]),
                            "achieved_GBs": round(gbs, 1),
                            "frac": round(gbs / PEAK_HBM_GBS, 4)})

    result = {
        "value": round(B / (step_ms * 1e-3), 1),
        "unit": "samples/s",
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(step_ms, 4),
        "config": {"workload": desc, "global_batch": B, "parallelism": "single GPU",
                   "params": int(sum(p.size for p in params)),
                   "step_tflops": round(flops_fn(cfg) / (step_ms * 1e-3) / 1e12, 2),
                   "execution": ("captured fwd+bwd HIP graph replay + eager fused Adam, every step"
                                 if graph else "eager launches on one stream"),
                   "wall_s_timed_region": round(wall, 3)},
        "roofline": ({"bound": "mfma", "kernel": KERNEL_CLASS.get(config, DEFAULT_KERNEL_CLASS),
                     "achieved": round(achieved, 2), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
                     "traffic": PMC_TRAFFIC_BYTES.get(config),
                     "traffic_unit": "bytes per launch (rocprofv3 PMC, see profiles/)",
                     "launches_per_step": launches.value // prof_steps,
                     "avg_launch_us": round(per_launch_us, 2),
                     "flops_per_launch": flops_per_launch,
                     "share_of_step": round(gemm_share, 3)}
                     if launches.value else small_roofline(hbm_kernels, step_ms, config)),
        "hbm_kernels": ({"peak_GBs": PEAK_HBM_GBS,
                         "note": "algorithmic bytes (inputs read once, outputs written once) / "
                                 "event-timed launch duration, per bandwidth-bound kernel",
                         "kernels": hbm_kernels} if hbm_detail else
                        {"top": [{k: r[k] for k in ("kernel", "launches_per_step", "avg_us", "frac")}
                                 for r in hbm_kernels[:4]]}),
    }
    if loader and config != 5:
        modes = ["resident", "stream"] if loader == "both" else [loader]
        result["loader"] = [loader_leg(sess, cfg, B, steps, step_ms, m) for m in modes]
    sess.close()
    return result


EXTRA_STEPS = {1: 200, 3: 20, 4: 20, 5: 20}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--steps", type=int, default=None, help="default 50 (config 1: 200)")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--only", action="store_true",
                    help="measure only --config; by default the other four configs are also timed "
                         "(GPU legs only, 20 steps each after 5 warm-up steps; config 1: 200) and "
                         "reported under 'other_configs'")
    ap.add_argument("--graph", action="store_true",
                    help="replay the step's zero_grad + forward + loss + backward as one captured "
                         "HIP graph (cnt_capture_step), Adam eagerly after it; same results bit for "
                         "bit, measured no faster on MI355X (the cost per kernel is GPU-side)")
    ap.add_argument("--layer-by-layer", action="store_true",
                    help="run config 1's step layer by layer (seven launches) instead of the fused "
                         "two-launch step (cnt_set_fused_step off); other configs have no fused step")
    ap.add_argument("--traffic-calibration", action="store_true",
                    help="only run the known-traffic reference kernel (cnhip_add over 64 Mi floats, "
                         "5 times: 512 MiB read + 256 MiB written per launch) that scales the PMC "
                         "FETCH_SIZE / WRITE_SIZE counts behind roofline.traffic")
    ap.add_argument("--loader", choices=["resident", "stream", "both"], default=None,
                    help="also time the same steps fed by the DataLoader (configs 1-4): 'resident' "
                         "gathers each batch in HBM, 'stream' uploads it from page-locked host "
                         "memory on a copy stream; reported under 'loader', never as 'value'")
    ap.add_argument("--phase-stamps", action="store_true",
                    help="only time the phases of config 4's persistent LSTM timesteps "
                         "(cnhip_lstm_phase_stamps) and print them as JSON")
    args = ap.parse_args()
    if args.traffic_calibration:
        return traffic_calibration()
    if args.phase_stamps:
        return phase_stamps(4)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (got --gpus {args.gpus}); the "
              "multi-GPU data-parallel design is described, not built", file=sys.stderr)
        return 2
    steps = args.steps if args.steps is not None else (200 if args.config == 1 else 50)

    from cppnet_amd import _capi

    lib = _capi.load()
    if lib.cnhip_device_count() < 1:
        log("bench.py: no GPU visible")
        return 1
    try:
        head = measure(args.config, steps, args.warmup, args.graph, args.loader,
                       fused=not args.layer_by_layer)
    except RuntimeError as e:
        log(f"bench.py: {e}")
        return 1
    result = {"metric": METRIC, "value": head["value"], "unit": head["unit"], "n_gpus": 1,
              "steps": steps, "warmup": args.warmup, "ms_per_step": head["ms_per_step"],
              "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
              "data": "synthetic (seeded inputs/labels, reference init distributions; resident in HBM)"}
    result.update({k: v for k, v in head.items() if k not in ("value", "unit", "steps", "warmup",
                                                                "ms_per_step")})
    result["cpu_baseline"] = None
    if not args.only:
        others = {}
        for c in (1, 2, 3, 4, 5):
            if c == args.config:
                continue
            try:
                r = measure(c, EXTRA_STEPS.get(c, 20), 5, args.graph, None, hbm_detail=False,
                            fused=not args.layer_by_layer)
            except RuntimeError as e:
                log(f"bench.py: {e}")
                return 1
            others[str(c)] = {"value": r["value"], "unit": r["unit"], "ms_per_step": r["ms_per_step"],
                              "steps": r["steps"], "warmup": r["warmup"],
                              "workload": r["config"]["workload"],
                              "global_batch": r["config"]["global_batch"],
                              "step_tflops": r["config"]["step_tflops"],
                              "roofline": r["roofline"], "hbm_kernels_top": r["hbm_kernels"]["top"]}
        result["other_configs"] = others
    if not args.no_cpu_baseline:
        try:
            result["cpu_baseline"] = cpu_baseline(args.config, args.cpu_seconds)
        except Exception as e:  # the GPU figure stands on its own
            log(f"bench.py: cpu baseline failed: {e!r}")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
