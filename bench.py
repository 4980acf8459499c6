#!/usr/bin/env python3
"""Benchmark of the MI355X GEMM hot path (BASELINE.json metric).

Step = one bf16-storage 4096^3 product C = A @ B through ``amd.matmul``, the
call Tensor ``@`` makes (fp32 accumulation; the result keeps A's storage
dtype, bf16, as the reference's matmul does; BASELINE config 2, the largest
single-GPU config the headline is quoted on).  The same product with an fp32
output through ``gemm`` is reported beside it.  W untimed warm-up steps, then K steps
timed with HIP events on the default stream (the stream every kernel runs
on) between two device synchronisations.  The JSON line also carries the
other configs (fp32 4096^3, the ragged shape, attention bmm and fused
attention, dense Linear fwd/bwd, MoE grouped experts) measured the same way, the roofline of the
dominant kernel and the CPU baseline (the pure-Python float64 restatement
of the reference CPU GEMM, timed on a bounded sample on this host).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only NAME]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from array import array
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "TFLOP/s + % MFMA peak: fp32/bf16 GEMM 4096^3, attention bmm, MoE grouped GEMM"
PEAK = {"bf16": 2516.6, "fp32": 157.3}  # dense MFMA TFLOP/s of MI355X (AMD spec)
HBM_PEAK = 8000.0  # GB/s


def upload(x, dtype):
    from qutai_amd.backends import amd

    return amd.storage(array("f", np.ascontiguousarray(x, dtype=np.float32).tobytes()), dtype=dtype)


class Timer:
    """HIP events on the default stream around a block of launches."""

    def __init__(self, runtime):
        self.runtime = runtime
        self.start, self.end = runtime.event(), runtime.event()

    def time(self, fn, steps, warmup, warm_seconds=0.3):
        # W warm-up steps, then more untimed steps until the GPU has been busy
        # for warm_seconds (clocks settle; the first launches run slower)
        for _ in range(warmup):
            fn()
        self.runtime.synchronize()
        begin = time.perf_counter()
        while time.perf_counter() - begin < warm_seconds:
            for _ in range(4):
                fn()
            self.runtime.synchronize()
        wall = time.perf_counter()
        self.runtime.record(self.start)
        for _ in range(steps):
            fn()
        self.runtime.record(self.end)
        self.runtime.synchronize()
        wall = time.perf_counter() - wall
        return self.runtime.elapsed_ms(self.start, self.end) / steps, wall * 1e3 / steps


# ---- workloads -----------------------------------------------------------------

def gemm_square(dtype, n=4096, seed=1, out_dtype=None):
    """C = A @ B, 4096^3 row-major.  By default through ``amd.matmul``, the
    call Tensor ``@`` makes: the output has the storage dtype of A, as in the
    reference (src/qutai/backends/cuda.py:374, ``out_dtype=left.dtype``), so
    bf16 storage gives a bf16 result of the fp32 accumulation.  With
    ``out_dtype`` the product goes through ``amd.gemm`` into a preallocated
    output of that dtype (the reference's ``gemm`` default is fp32)."""
    from qutai_amd.backends import amd

    rng = np.random.default_rng(seed)
    a = upload(rng.standard_normal(n * n) * n ** -0.5, dtype)
    b = upload(rng.standard_normal(n * n) * n ** -0.5, dtype)
    flops = 2.0 * n ** 3
    config = {"M": n, "N": n, "K": n, "storage": dtype, "layout": "row-major A@B (NN)"}
    if out_dtype is None:
        return (lambda: amd.matmul(a, b, (n, n), (n, n))), flops, {**config, "out": dtype, "call": "Tensor @"}
    out = amd.full(n * n, 0.0, dtype=out_dtype)
    return ((lambda: amd.gemm(a, b, n, n, n, out=out, out_dtype=out_dtype)), flops,
            {**config, "out": out_dtype, "call": "gemm"})


def gemm_ragged(dtype, seed=1, order="MNK"):
    """BASELINE's ragged edge shape 4095x4097x1000 in both axis orders: "MNK"
    reads it as M x N x K (A 4095x1000, B 1000x4097, a 4095x4097 output),
    "MKN" as the reference's (rows, inner, cols) convention (A 4095x4097,
    B 4097x1000, a 4095x1000 output).  fp32 output through ``amd.gemm``
    (the reference gemm's default)."""
    from qutai_amd.backends import amd

    m, n, k = (4095, 4097, 1000) if order == "MNK" else (4095, 1000, 4097)
    rng = np.random.default_rng(seed)
    a = upload(rng.standard_normal(m * k) * k ** -0.5, dtype)
    b = upload(rng.standard_normal(k * n) * k ** -0.5, dtype)
    out = amd.full(m * n, 0.0, dtype="float32")
    return ((lambda: amd.gemm(a, b, m, k, n, out=out)), 2.0 * m * n * k,
            {"M": m, "N": n, "K": k, "storage": dtype, "axis_order": order})


def attention_bmm(seed=2):
    """S = Q K^T (NT, batched 128), P = softmax(S / 8) rows, O = P V (NN)."""
    from qutai_amd.backends import amd

    b, h, t, d = 8, 16, 2048, 64
    rng = np.random.default_rng(seed)
    q = upload(rng.standard_normal(b * h * t * d), "bfloat16")
    k = upload(rng.standard_normal(b * h * t * d), "bfloat16")
    v = upload(rng.standard_normal(b * h * t * d), "bfloat16")
    s = amd.full(b * h * t * t, 0.0, dtype="bfloat16")
    o = amd.full(b * h * t * d, 0.0, dtype="bfloat16")

    def step():
        amd.gemm(q, k, t, d, t, batch=b * h, transpose_right=True, out_dtype="bfloat16", out=s)
        p = amd.softmax(s, (b * h * t, t), -1, scale=d ** -0.5)
        amd.gemm(p, v, t, t, d, batch=b * h, out_dtype="bfloat16", out=o)

    # algorithmic HBM bytes of the three launches: S written (Q, K read),
    # S read and P written, P read (V read, O written); bf16 throughout
    scores, rows = b * h * t * t * 2, b * h * t * d * 2
    hbm_bytes = (scores + 2 * rows) + 2 * scores + (scores + 2 * rows)
    return step, 2 * 2.0 * b * h * t * t * d, {"batch": b, "heads": h, "seq": t, "head_dim": d, "storage": "bfloat16",
                                               "hbm_bytes": hbm_bytes}


def attention_fused(seed=2, causal=False):
    """Score and value products in one fused kernel (S never stored): config 3
    shape in the nn layout [B][H][T][D] non-causal, or the lm layout
    [B][T][H][D] causal (the lm path, algorithmic FLOPs of the visible half)."""
    from qutai_amd.backends import amd_lm

    b, h, t, d = 8, 16, 2048, 64
    rng = np.random.default_rng(seed)
    q, k, v = (upload(rng.standard_normal(b * h * t * d), "bfloat16") for _ in range(3))
    layout = 1 if causal else 0

    def step():
        amd_lm.attention(q, k, v, b, t, h, h, d, causal=causal, layout=layout)

    pairs = t * (t + 1) / 2 if causal else t * t
    return step, 2 * 2.0 * b * h * pairs * d, {"batch": b, "heads": h, "seq": t, "head_dim": d,
                                                "storage": "bfloat16", "causal": causal,
                                                "layout": "B,T,H,D" if causal else "B,H,T,D"}


def attention_fused_backward(seed=2):
    """Fused causal attention backward in the lm layout at the config 3 shape:
    dq (recomputing P) then dk/dv; algorithmic FLOPs = the five products
    S, dP, dQ, dK, dV over the visible half."""
    from qutai_amd.backends import amd_lm

    b, h, t, d = 8, 16, 2048, 64
    rng = np.random.default_rng(seed)
    q, k, v, g = (upload(rng.standard_normal(b * h * t * d), "bfloat16") for _ in range(4))
    out, lse = amd_lm.attention(q, k, v, b, t, h, h, d)

    def step():
        amd_lm.attention_backward(g, q, k, v, out, lse, b, t, h, h, d)

    return step, 5 * 2.0 * b * h * (t * (t + 1) / 2) * d, {"batch": b, "heads": h, "seq": t, "head_dim": d,
                                                            "storage": "bfloat16", "causal": True,
                                                            "layout": "B,T,H,D"}


def dense_linear(seed=3):
    """SwiGLU projections of a 4096-token batch: Y = X W^T, dX = dY W, dW = dY^T X (x3)."""
    from qutai_amd.backends import amd

    tokens, width, hidden = 4096, 2048, 5632
    rng = np.random.default_rng(seed)
    x = upload(rng.standard_normal(tokens * width), "bfloat16")
    w_in = [upload(rng.standard_normal(hidden * width) * 0.02, "bfloat16") for _ in range(2)]
    w_down = upload(rng.standard_normal(width * hidden) * 0.02, "bfloat16")
    g_hidden = upload(rng.standard_normal(tokens * hidden), "bfloat16")
    h_act = upload(rng.standard_normal(tokens * hidden), "bfloat16")
    g_out = upload(rng.standard_normal(tokens * width), "bfloat16")

    def step():
        for w in w_in:  # gate / up: X [T,d] W^T [h,d]
            amd.gemm(x, w, tokens, width, hidden, transpose_right=True, out_dtype="bfloat16")
            amd.gemm(g_hidden, w, tokens, hidden, width, out_dtype="bfloat16")
            amd.gemm(g_hidden, x, hidden, tokens, width, transpose_left=True, out_dtype="bfloat16")
        amd.gemm(h_act, w_down, tokens, hidden, width, transpose_right=True, out_dtype="bfloat16")
        amd.gemm(g_out, w_down, tokens, width, hidden, out_dtype="bfloat16")
        amd.gemm(g_out, h_act, width, tokens, hidden, transpose_left=True, out_dtype="bfloat16")

    return step, 9 * 2.0 * tokens * width * hidden, {"tokens": tokens, "d_model": width, "ffn": hidden,
                                                      "storage": "bfloat16", "gemms": 9}


def moe_experts(seed=4):
    """Routing + gather + grouped gate/up/down + SiLU*up + combine (forward)."""
    from qutai_amd.backends import amd
    from qutai_amd.backends import amd_lm

    tokens, width, experts, hidden, top_k = 8192, 2048, 8, 1408, 2
    rng = np.random.default_rng(seed)
    x = upload(rng.standard_normal(tokens * width), "bfloat16")
    logits = upload(rng.standard_normal(tokens * experts), "float32")
    w_gate = upload(rng.standard_normal(experts * hidden * width) * 0.02, "bfloat16")
    w_up = upload(rng.standard_normal(experts * hidden * width) * 0.02, "bfloat16")
    w_down = upload(rng.standard_normal(experts * width * hidden) * 0.02, "bfloat16")

    def step():
        route = amd_lm.routing(logits, tokens, experts, top_k, download_counts=False)
        amd_lm.moe_experts_forward(x, route, w_gate, w_up, w_down, width, hidden)

    flops = 2.0 * tokens * top_k * 3 * width * hidden
    return step, flops, {"tokens": tokens, "d_model": width, "experts": experts, "top_k": top_k,
                         "hidden": hidden, "storage": "bfloat16"}


def moe_train(seed=4):
    """Config 5 MoE forward + backward through the SparseMoE layer (routing,
    gather, grouped gate/up/down, combine; backward: combine backward,
    grouped data-gradient GEMMs, grouped-K weight-gradient GEMMs, routing
    backward, router Linear backward)."""
    from qutai_amd import Tensor
    from qutai_amd.backends import amd
    from qutai_amd.lm.layers import SparseMoE

    from qutai_amd.backends import amd_lm

    tokens, width, experts, hidden, top_k = 8192, 2048, 8, 1408, 2
    rng = np.random.default_rng(seed)
    # random init from numpy draws (69 M Random.gauss draws in CPython would
    # take a minute); same shapes and scales as the layer's own init
    host_normal = amd_lm.normal
    amd_lm.normal = lambda size, mean=0.0, std=1.0, *, seed=None, dtype="float32": upload(
        rng.normal(mean, std, size), dtype)
    try:
        layer = SparseMoE(width, hidden, experts, top_k, dtype="bfloat16", seed=seed)
    finally:
        amd_lm.normal = host_normal
    x = Tensor(upload(rng.standard_normal(tokens * width), "bfloat16"), shape=(tokens, width), requires_grad=True)
    g = Tensor(upload(rng.standard_normal(tokens * width), "bfloat16"), shape=(tokens, width))

    def step():
        for p in (x, *layer.parameters()):
            p.grad = None
        y, aux = layer(x)
        y.backward(g)

    flops = 9 * 2.0 * tokens * top_k * width * hidden
    return step, flops, {"tokens": tokens, "d_model": width, "experts": experts, "top_k": top_k,
                         "hidden": hidden, "storage": "bfloat16", "pass": "forward+backward"}


def decoder_train(seed=5):
    """One Decoder.loss forward + backward under autocast on config 4's
    shapes (4096 tokens = 2 x 2048, d_model 2048, 32 heads of 64 with 8 KV
    heads, SwiGLU 5632, vocab 32768, 2 layers, chunked head of 1024 rows):
    embedding, RMSNorm, RoPE, fused attention, the 9 projection GEMMs per
    layer, the loss head and every backward kernel.  FLOPs: 6 x matmul
    parameters x tokens plus causal attention (fwd 2 T^2 D H per sequence,
    backward twice that)."""
    from qutai_amd.backends import amd_lm
    from qutai_amd.lm import Config, Decoder, autocast

    config = Config(vocab_size=32768, n_layers=2, d_model=2048, n_heads=32, n_kv_heads=8, d_ff=5632,
                    max_seq_len=2048, activation_checkpointing=False)
    batch, time_ = 2, 2048
    rng = np.random.default_rng(seed)
    host_normal = amd_lm.normal
    amd_lm.normal = lambda size, mean=0.0, std=1.0, *, seed=None, dtype="float32": upload(
        rng.normal(mean, std, size), dtype)
    try:
        model = Decoder(config, seed=seed)
    finally:
        amd_lm.normal = host_normal
    tokens = rng.integers(0, config.vocab_size, size=(batch, time_)).tolist()
    params = model.parameters()

    def step():
        for p in params:
            p.grad = None
        with autocast():
            loss = model.loss(tokens, chunk_size=1024)
        loss.backward()

    d, kv = config.d_model, config.n_kv_heads * (config.d_model // config.n_heads)
    matmul_params = config.n_layers * (2 * d * d + 2 * d * kv + 3 * d * config.d_ff) + config.vocab_size * d
    n_tokens = batch * time_
    attention = config.n_layers * batch * 3 * 2 * time_ * time_ * d
    flops = 6.0 * matmul_params * n_tokens + attention
    return step, flops, {"tokens": n_tokens, "batch": batch, "seq_len": time_, "d_model": d, "n_layers": 2,
                         "heads": 32, "kv_heads": 8, "d_ff": config.d_ff, "vocab": config.vocab_size,
                         "storage": "fp32 weights, bf16 activations (autocast)", "pass": "loss forward+backward"}


WORKLOADS = {
    "gemm_bf16_4096": (lambda: gemm_square("bfloat16"), "bf16"),
    "gemm_bf16_4096_f32out": (lambda: gemm_square("bfloat16", out_dtype="float32"), "bf16"),
    "gemm_fp32_4096": (lambda: gemm_square("float32"), "fp32"),
    "gemm_bf16_ragged": (lambda: gemm_ragged("bfloat16"), "bf16"),
    "gemm_fp32_ragged": (lambda: gemm_ragged("float32"), "fp32"),
    "gemm_bf16_ragged_mkn": (lambda: gemm_ragged("bfloat16", order="MKN"), "bf16"),
    "gemm_fp32_ragged_mkn": (lambda: gemm_ragged("float32", order="MKN"), "fp32"),
    "attention_bmm": (attention_bmm, "bf16"),
    "attention_fused": (attention_fused, "bf16"),
    "attention_fused_causal": (lambda: attention_fused(causal=True), "bf16"),
    "attention_fused_backward": (attention_fused_backward, "bf16"),
    "dense_linear_fwd_bwd": (dense_linear, "bf16"),
    "moe_grouped": (moe_experts, "bf16"),
    "moe_train": (moe_train, "bf16"),
    "decoder_train": (decoder_train, "bf16"),
}
HEADLINE = "gemm_bf16_4096"


def traffic_from_profiles(name):
    """HBM bytes per launch of the headline kernel, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, copy-kernel scaled)."""
    path = ROOT / "profiles" / f"{name}_traffic.md"
    if not path.exists():
        return None
    match = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", path.read_text())
    return float(match.group(1)) if match else None


def cpu_baseline(seconds_target=15.0):
    """Pure-Python float64 restatement of the reference CPU GEMM
    (src/qutai/backends/cpu.py:152-162) on the first rows of the 4096^3
    product, one core; scaled to TFLOP/s by the FLOPs of the sample."""
    from oracle import reference as ora

    n = 4096
    rng = np.random.default_rng(1)
    a = (rng.standard_normal(n * n) * n ** -0.5).astype(np.float32).astype(np.float64)
    b = (rng.standard_normal(n * n) * n ** -0.5).astype(np.float32).astype(np.float64)
    left_rows = a.reshape(n, n)
    right = b.tolist()
    rows = 1
    elapsed = 0.0
    done_rows = 0
    while elapsed < seconds_target and done_rows < 64:
        sample = left_rows[done_rows:done_rows + rows].ravel().tolist()
        start = time.perf_counter()
        ora.matmul(sample, right, (rows, n), (n, n))
        elapsed += time.perf_counter() - start
        done_rows += rows
    flops = 2.0 * done_rows * n * n
    return {"value": flops / elapsed / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"first {done_rows} rows of C = A@B, 4096^3 float64 (cpu.matmul restated, oracle/reference.py),"
                      f" {flops / 1e9:.2f} GFLOP in {elapsed:.1f} s on 1 of {os.cpu_count()} host cores"}


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--only", default=None, help="run one workload")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--calibrate-copy", action="store_true",
                        help="run only a plain 256 MiB copy kernel (the HBM-counter calibration for rocprofv3 --pmc)")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the GEMM path is single-device (see DESIGN.md for how it would shard)",
              file=sys.stderr)
        sys.exit(2)

    from qutai_amd.backends import amd

    runtime = amd.get_runtime()
    if args.calibrate_copy:
        count = 64 * 1024 * 1024  # fp32 values: 256 MiB read + 256 MiB written per launch
        src, dst = amd.full(count, 1.5, dtype="float32"), amd.full(count, 0.0, dtype="float32")
        for _ in range(3):
            runtime.call("qutai_amd_cast", src.ptr, dst.ptr, count, 0, 0)
        runtime.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": count * 4, "bytes_written": count * 4}))
        return
    timer = Timer(runtime)
    names = [args.only] if args.only else list(WORKLOADS)
    results = {}
    for name in names:
        make, kind = WORKLOADS[name]
        try:
            fn, flops, config = make()
        except (AttributeError, ImportError, NotImplementedError) as error:
            results[name] = {"error": f"not available: {error}"}
            continue
        steps = args.steps if name == HEADLINE else max(3, args.steps // 2)
        ms, wall_ms = timer.time(fn, steps, args.warmup)
        tflops = flops / (ms * 1e-3) / 1e12
        results[name] = {"ms": round(ms, 4), "wall_ms": round(wall_ms, 4), "tflops": round(tflops, 1),
                         "peak_frac": round(tflops / PEAK[kind], 4), "dtype": kind, **config}
        if "hbm_bytes" in config:  # HBM-bound workloads: the fraction of the 8 TB/s roofline
            rate = config["hbm_bytes"] / (ms * 1e-3)
            results[name].update(hbm_tbps=round(rate / 1e12, 3), hbm_frac=round(rate / 1e9 / HBM_PEAK, 4))
        print(f"# {name}: {ms * 1e3:.1f} us/step  {tflops:.1f} TFLOP/s  ({100 * tflops / PEAK[kind]:.1f}% of "
              f"{kind} peak)", file=sys.stderr, flush=True)
        del fn
    head = results.get(HEADLINE, {})
    ms = head.get("ms")
    value = head.get("tflops")
    traffic = traffic_from_profiles(HEADLINE)
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (numpy PCG64 draws, N(0,1)*K^-1/2, seed 1); inputs resident in HBM",
        "config": {"workload": HEADLINE, "M": 4096, "N": 4096, "K": 4096, "storage": "bfloat16",
                   "accumulate": "float32", "out": "bfloat16", "call": "Tensor @ (amd.matmul)",
                   "layout": "row-major A@B"},
        "roofline": None,
        "results": results,
    }
    if value is not None:
        line["roofline"] = {"bound": "mfma", "achieved": value, "peak": PEAK["bf16"], "unit": "TFLOP/s",
                            "frac": round(value / PEAK["bf16"], 4), "traffic": traffic,
                            "kernel": "pingpong_entry<PingPong<bf16 NN>> (256x256 tile, 8 waves in two phase "
                                      "groups, BK 64, direct-to-LDS A/B rings)",
                            "algorithmic_flops_per_launch": 2 * 4096 ** 3}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
