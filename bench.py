#!/usr/bin/env python3
"""Benchmark of tensorsmith's attention hot path on one MI355X.

Headline workload (one "step"): causal self-attention forward + backward,
B=16 H=16 S=2048 D=128, bf16 inputs, fp32 accumulate/softmax, row LSE saved,
through the public API (``scaled_dot_product_attention(..., is_causal=True)``
then ``backward``).  Inputs are synthetic (seeded N(0,1) * 0.5 in bf16, dO
N(0,1)) and resident in HBM before timing starts.

``value`` is algorithmic TFLOP/s: causal forward 4*B*H*S^2*D/2 FLOP and
backward 2.5x that (FlashAttention counting), divided by the measured step
time.  The JSON line also carries

* ``roofline`` -- the dominant kernel's achieved rate (algorithmic work per
  launch / its mean duration from HIP events recorded on its own stream
  during the timed steps) against the MI355X dense bf16 MFMA peak;
* ``variants`` -- the headline step with a general [S, S] boolean mask,
  with dropout p = 0.1, and with RoPE folded into the kernels;
* ``decode`` -- KV-cache decode (B=64 H=32 D=128 fp16 cache, lengths
  U[512, 8192]): tokens/s and HBM GB/s with its own roofline;
* ``prefill`` -- long-context causal prefill with a key-padding mask
  (B=2 H=32 S=32768 D=128 bf16, valid lengths U[16384, 32768]), forward
  only: TFLOP/s over the exact unmasked (query, key) pairs and its fraction
  of the bf16 peak;
* ``lm_step`` -- a 6-layer decoder LM (d_model 512, 8 heads, FFN 2048 GELU,
  pre-LayerNorm, learned positions, vocab 32000), fp16 autocast, forward +
  backward of next-token cross-entropy at batch 8 x 1024 tokens: step time,
  tokens/s and the share of the step spent in the attention kernels;
* ``cached_step`` -- one cached MultiHeadAttention decode step (E 4096,
  32 / 8 heads of 128, fp16, batch 64, 1024 cached positions) with the
  projections, RoPE and K/V append in one kernel, against the same module
  with that kernel switched off, and the fused kernel's HBM rate;
* ``fp32`` -- causal fp32 forward + backward on the generic kernels at the
  reference's CPU-runnable shape (B=8 H=4 S=256 D=64) and at B=2 H=16
  S=2048 D=128: step time, TFLOP/s and the fraction of the fp32 peak;
* ``cpu_baseline`` -- the NumPy oracle (a restatement of the reference's
  streaming algorithm) on a bounded sample of the same inputs, on this
  host's cores.

Run ``python bench.py`` (defaults: 1 GPU, 20 steps, 5 warmup).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "custom-ml-library_amd"))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E
PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 (MFMA)
B, H, S, D = 16, 16, 2048, 128
DEC_B, DEC_H, DEC_D, DEC_CAP, DEC_LO, DEC_HI = 64, 32, 128, 8192, 512, 8192
PF_B, PF_H, PF_S, PF_D, PF_LO = 2, 32, 32768, 128, 16384
LONG_B, LONG_H, LONG_S = 16, 16, 8192
LM_LAYERS, LM_DIM, LM_HEADS, LM_FFN, LM_VOCAB, LM_B, LM_S = 6, 512, 8, 2048, 32000, 8, 1024
ATTN_KERNELS = ("fwd_mfma", "bwd_dkdv_mfma", "bwd_dq_ds", "bwd_dq_mfma", "bwd_rows", "generic_fwd",
                "generic_bwd_delta", "generic_bwd_dq", "generic_bwd_dkdv", "key_mask_lengths",
                "decode_split", "decode_merge", "rope")


def causal_fwd_flops(b, h, s, d):
    return 4.0 * b * h * s * s * d / 2


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--decode-steps", type=int, default=50)
    ap.add_argument("--cpu-batches", type=int, default=4,
                    help="batch rows (of 16 heads each) in the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--workload",
                    choices=["all", "fwd_bwd", "variants", "decode", "decode_int8", "prefill", "lm",
                             "cached_step", "fp32", "d32", "long", "copy"],
                    default="all",
                    help="run one workload only (for profiling); 'all' prints the contract line")
    return ap.parse_args()


def traffic_for(kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 --pmc summary."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    entry = json.loads(path.read_text()).get(kernel)
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def bench_fwd_bwd(ts, torch, steps, warmup):
    from tensorsmith_hip import _lib

    gen = torch.Generator(device="cuda").manual_seed(42)

    def draw(scale):
        x = torch.randn((B, H, S, D), generator=gen, device="cuda", dtype=torch.float32)
        return (x * scale).to(torch.bfloat16)

    q_raw, k_raw, v_raw, g_raw = draw(0.5), draw(0.5), draw(0.5), draw(1.0)
    q, k, v = (ts.Tensor(t, device="hip", requires_grad=True) for t in (q_raw, k_raw, v_raw))
    upstream = ts.Tensor(g_raw, device="hip")

    def step():
        for t in (q, k, v):
            t.zero_grad()
        out = ts.nn.scaled_dot_product_attention(q, k, v, is_causal=True)
        out.backward(upstream)
        return out

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    if _lib.last_kernel_path() != _lib.PATH_MFMA:
        raise RuntimeError("the MFMA kernels did not run for the headline workload")
    _lib.profile_reset()
    _lib.profile_enable(True)
    # per-step GPU times from events between the steps (the reference's
    # timing contract reports the median and p95 of the repeats,
    # benchmarks/common.py:24-64); `value` stays whole-run wall time / steps
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    marks[0].record()
    for i in range(steps):
        step()
        marks[i + 1].record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.profile_enable(False)
    kernels = _lib.profile_read()
    step_ms = sorted(marks[i].elapsed_time(marks[i + 1]) for i in range(steps))
    fwd = causal_fwd_flops(B, H, S, D)
    flops = fwd * 3.5
    ms = elapsed / steps * 1e3
    # algorithmic FLOP per launch: forward kernel = QK^T + PV (2 GEMMs);
    # dK/dV kernel = S recompute, dP, dV, dK (4 of the backward's 5 GEMMs);
    # dQ kernel = dQ (1 GEMM: from the stored dS, or with an S / dP recompute
    # that is overhead, not counted)
    work = {"fwd_mfma": fwd, "bwd_dkdv_mfma": 2.0 * fwd, "bwd_dq_ds": 0.5 * fwd,
            "bwd_dq_mfma": 0.5 * fwd}
    per_kernel = {n: {"launches": c, "mean_ms": t / max(c, 1)} for n, (c, t) in kernels.items()}
    dom = max((n for n in per_kernel if n in work), key=lambda n: per_kernel[n]["mean_ms"])
    achieved = work[dom] / (per_kernel[dom]["mean_ms"] * 1e-3) / 1e12
    for n, w in work.items():
        if n in per_kernel:
            per_kernel[n]["tflops"] = round(w / (per_kernel[n]["mean_ms"] * 1e-3) / 1e12, 1)
    result = {
        "ms_per_step": ms,
        "step_ms": {"mean": round(statistics.fmean(step_ms), 4),
                    "median": round(statistics.median(step_ms), 4),
                    "p95": round(step_ms[min(steps - 1, math.ceil(0.95 * steps) - 1)], 4),
                    "min": round(step_ms[0], 4), "max": round(step_ms[-1], 4)},
        "value": flops / (ms * 1e-3) / 1e12,
        "kernels": {n: {k_: (round(v_, 4) if isinstance(v_, float) else v_) for k_, v_ in d.items()}
                    for n, d in per_kernel.items()},
        "roofline": {
            "kernel": dom, "bound": "mfma", "achieved": round(achieved, 1),
            "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic_for(dom),
        },
    }
    host = {"q": q_raw, "k": k_raw, "v": v_raw, "g": g_raw}
    return result, host


def bench_variants(ts, torch, steps, warmup, host, rounds=3):
    """The headline shape again through the other MFMA kernel variants: a
    general [S, S] boolean mask (with the causal flag), dropout p = 0.1 on the
    hip backend, and RoPE folded into the kernels (unrotated q / k, as
    MultiHeadAttention calls it).  Same FLOP count per step as the headline.
    The plain causal step runs in the same leg and the cases take turns over
    `rounds` rounds of `steps` steps (medians reported), so each ratio to the
    plain step compares runs at the same clocks."""
    q, k, v = (ts.Tensor(host[n], device="hip", requires_grad=True) for n in ("q", "k", "v"))
    upstream = ts.Tensor(host["g"], device="hip")
    tril = ts.Tensor(torch.ones((S, S), dtype=torch.bool, device="cuda").tril(), device="hip")
    cases = {
        "plain": dict(is_causal=True),
        "general_bool_mask": dict(attn_mask=tril, is_causal=True),
        "dropout_p0.1": dict(is_causal=True, dropout_p=0.1, backend="hip"),
        "rope_folded": dict(is_causal=True, _rope=(0, 0, 10000.0)),
    }
    from tensorsmith_hip import _lib

    flops = causal_fwd_flops(B, H, S, D) * 3.5

    def step(kw):
        for t in (q, k, v):
            t.zero_grad()
        ts.nn.scaled_dot_product_attention(q, k, v, **kw).backward(upstream)

    times = {name: [] for name in cases}
    for r in range(rounds):
        for name, kw in cases.items():
            for _ in range(warmup if r == 0 else 1):
                step(kw)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                step(kw)
            torch.cuda.synchronize()
            times[name].append((time.perf_counter() - t0) / steps * 1e3)
    out = {}
    for name, kw in cases.items():
        _lib.profile_reset()
        _lib.profile_enable(True)
        for _ in range(2):
            step(kw)
        torch.cuda.synchronize()
        _lib.profile_enable(False)
        kernels = {n: round(t / max(c, 1), 4) for n, (c, t) in _lib.profile_read().items()}
        ms = statistics.median(times[name])
        out[name] = {"ms_per_step": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                     "kernel_ms": kernels}
    for name in cases:
        out[name]["vs_plain"] = round(out[name]["ms_per_step"] / out["plain"]["ms_per_step"], 3)
    return out


def bench_decode(ts, torch, steps, warmup):
    from tensorsmith_hip import _lib

    gen = torch.Generator(device="cuda").manual_seed(42)
    shape = (DEC_B, DEC_H, DEC_CAP, DEC_D)
    q_raw = torch.randn((DEC_B, DEC_H, 1, DEC_D), generator=gen, device="cuda").half()
    k_raw = torch.randn(shape, generator=gen, device="cuda", dtype=torch.float16)
    v_raw = torch.randn(shape, generator=gen, device="cuda", dtype=torch.float16)
    lengths = torch.randint(DEC_LO, DEC_HI + 1, (DEC_B,), generator=gen, device="cuda")
    keymask = torch.arange(DEC_CAP, device="cuda")[None, :] < lengths[:, None]
    q, k, v = (ts.Tensor(t, device="hip") for t in (q_raw, k_raw, v_raw))
    mask = ts.Tensor(keymask[:, None, None, :], device="hip")

    def step():
        with ts.no_grad():
            return ts.nn.scaled_dot_product_attention(q, k, v, mask)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    if _lib.last_kernel_path() != _lib.PATH_DECODE:
        raise RuntimeError("the decode kernel did not run for the decode workload")
    _lib.profile_reset()
    _lib.profile_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.profile_enable(False)
    kernels = _lib.profile_read()
    lens = lengths.cpu().numpy()
    kv_bytes = float(lens.sum()) * DEC_H * DEC_D * 2 * 2
    qo_bytes = 2.0 * DEC_B * DEC_H * DEC_D * 2
    total_bytes = kv_bytes + qo_bytes
    ms = elapsed / steps * 1e3
    split_ms = kernels["decode_split"][1] / kernels["decode_split"][0]
    achieved = total_bytes / (split_ms * 1e-3) / 1e9
    return {
        "metric": "decode tokens/s",
        "value": DEC_B / (ms * 1e-3),
        "unit": "tokens/s",
        "ms_per_step": ms,
        "hbm_GBps_step": total_bytes / (ms * 1e-3) / 1e9,
        "bytes_per_step": total_bytes,
        "kernels": {n: {"launches": c, "mean_ms": round(t / max(c, 1), 4)}
                    for n, (c, t) in kernels.items()},
        "roofline": {
            "kernel": "decode_split", "bound": "hbm", "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": traffic_for("decode_split"),
        },
        "config": {"workload": "decode_f16_b64h32d128_len512_8192", "batch": DEC_B,
                   "heads": DEC_H, "head_dim": DEC_D, "cache_capacity": DEC_CAP,
                   "lengths": "U[512,8192] seeded", "sum_len": int(lens.sum())},
    }, {"q": q_raw, "k": k_raw, "v": v_raw, "lengths": lens}


def bench_decode_int8(ts, torch, steps, warmup, dec_inputs):
    """The decode workload over an int8 cache (the reference's quantised
    KVCache format): the same fp16 K/V, quantised once by the fused append
    kernel, then decoded with the int8 split-K kernel (dequantised inside),
    per-sequence lengths passed as kv_len."""
    import ctypes

    import numpy as np

    from tensorsmith_hip import _lib
    from tensorsmith_hip.nn.attention import _problem, _view

    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    q_raw, k_raw, v_raw = dec_inputs["q"], dec_inputs["k"], dec_inputs["v"]
    lens = dec_inputs["lengths"]
    shape = (DEC_B, DEC_H, DEC_CAP, DEC_D)
    k8, v8 = (torch.empty(shape, dtype=torch.int8, device="cuda") for _ in range(2))
    ks, vs = (torch.empty(shape[:3] + (1,), dtype=torch.float32, device="cuda") for _ in range(2))
    def append(src, codes, scales):
        _lib.check(lib.tsattn_kv_append_int8(_lib.F16, DEC_B, DEC_H, DEC_CAP, DEC_D,
                                             ctypes.byref(_view(src)), ctypes.byref(_view(codes)),
                                             ctypes.byref(_view(scales)), 0, stream), "append")

    for src, codes, scales in ((k_raw, k8, ks), (v_raw, v8, vs)):
        append(src, codes, scales)
    # the quantising append itself (whole cache, one tensor per launch), timed
    # with the library's HIP-event probes on its stream
    torch.cuda.synchronize()
    _lib.profile_reset()
    _lib.profile_enable(True)
    for _ in range(3):
        append(k_raw, k8, ks)
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    n_app, t_app = _lib.profile_read()["kv_append_int8"]
    app_ms = t_app / n_app
    app_bytes = float(DEC_B * DEC_H * DEC_CAP) * (DEC_D * 2 + DEC_D + 4)  # fp16 in, int8 + scale out
    kv_len = torch.as_tensor(lens.astype(np.int32), device="cuda")
    prob = _problem(DEC_B, DEC_H, DEC_H, 1, DEC_CAP, DEC_D, DEC_D, _lib.F16, 1 / math.sqrt(DEC_D),
                    False, 0)
    prob.kv_len = kv_len.data_ptr()
    out = torch.empty((DEC_B, DEC_H, 1, DEC_D), dtype=torch.float16, device="cuda")
    nbytes = lib.tsattn_decode_workspace(ctypes.byref(prob), 0)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    views = [ctypes.byref(_view(t)) for t in (q_raw, k8, v8, ks, vs, out)]

    def step():
        _lib.check(lib.tsattn_decode_forward_int8(ctypes.byref(prob), *views, 0,
                                                  ctypes.c_void_p(ws.data_ptr()), nbytes, stream),
                   "int8 decode")

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    _lib.profile_reset()
    _lib.profile_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.profile_enable(False)
    kernels = _lib.profile_read()
    kv_bytes = float(lens.sum()) * DEC_H * (DEC_D + 4) * 2  # int8 rows + fp32 scales, K and V
    total_bytes = kv_bytes + 2.0 * DEC_B * DEC_H * DEC_D * 2
    ms = elapsed / steps * 1e3
    split_ms = kernels["decode_split_int8"][1] / kernels["decode_split_int8"][0]
    achieved = total_bytes / (split_ms * 1e-3) / 1e9
    return {
        "metric": "decode tokens/s (int8 cache)",
        "value": DEC_B / (ms * 1e-3),
        "unit": "tokens/s",
        "ms_per_step": ms,
        "bytes_per_step": total_bytes,
        "kernels": {n: {"launches": c, "mean_ms": round(t / max(c, 1), 4)}
                    for n, (c, t) in kernels.items()},
        "roofline": {
            "kernel": "decode_split_int8", "bound": "hbm", "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBPS, 4),
        },
        "append": {
            "kernel": "kv_append_int8", "mean_ms": round(app_ms, 4), "bytes_per_launch": app_bytes,
            "roofline": {"bound": "hbm", "achieved": round(app_bytes / (app_ms * 1e-3) / 1e9, 1),
                         "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                         "frac": round(app_bytes / (app_ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)},
        },
        "config": {"workload": "decode_int8cache_f16q_b64h32d128_len512_8192", "batch": DEC_B,
                   "heads": DEC_H, "head_dim": DEC_D, "cache_capacity": DEC_CAP},
    }


def bench_prefill(ts, torch, steps, warmup):
    """Causal prefill over key-padded sequences; forward only (no grad)."""
    from tensorsmith_hip import _lib

    gen = torch.Generator(device="cuda").manual_seed(42)
    shape = (PF_B, PF_H, PF_S, PF_D)
    q, k, v = ((torch.randn(shape, generator=gen, device="cuda") * 0.5).to(torch.bfloat16)
               for _ in range(3))
    lengths = torch.randint(PF_LO, PF_S + 1, (PF_B,), generator=gen, device="cuda")
    keymask = (torch.arange(PF_S, device="cuda")[None, :] < lengths[:, None])[:, None, None, :]
    tq, tk, tv = (ts.Tensor(t, device="hip") for t in (q, k, v))
    tm = ts.Tensor(keymask, device="hip")

    def step():
        with ts.no_grad():
            return ts.nn.scaled_dot_product_attention(tq, tk, tv, tm, is_causal=True)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    if _lib.last_kernel_path() != _lib.PATH_MFMA:
        raise RuntimeError("the MFMA kernel did not run for the prefill workload")
    _lib.profile_reset()
    _lib.profile_enable(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.profile_enable(False)
    kernels = _lib.profile_read()
    # row i (< S) attends keys j <= i with j < L: min(i + 1, L) keys
    pairs = 0
    for L in lengths.cpu().tolist():
        pairs += L * (L + 1) // 2 + (PF_S - L) * L
    flops = 4.0 * PF_D * PF_H * pairs
    fwd_ms = kernels["fwd_mfma"][1] / kernels["fwd_mfma"][0]
    achieved = flops / (fwd_ms * 1e-3) / 1e12
    return {
        "ms_per_step": elapsed / steps * 1e3,
        "value": flops / (elapsed / steps) / 1e12,
        "unit": "TFLOP/s",
        "flop_per_step": flops,
        "kernels": {n: {"launches": c, "mean_ms": round(t / max(c, 1), 4)} for n, (c, t) in kernels.items()},
        "roofline": {"kernel": "fwd_mfma", "bound": "mfma", "achieved": round(achieved, 1),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4)},
        "config": {"workload": "causal_prefill_keypad_bf16_b2h32s32768d128", "batch": PF_B,
                   "heads": PF_H, "seq_len": PF_S, "head_dim": PF_D,
                   "lengths": [int(x) for x in lengths.cpu().tolist()]},
    }


def bench_long(ts, torch, steps, warmup):
    """Causal fwd+bwd at B16 H16 S8192 D128 bf16 through the public API: the
    stored dS of all heads (17.4 GB) exceeds the backward's 8 GiB region, so
    dK/dV and dQ-from-dS run over chunks of heads reusing one region (the
    launch counts of their probes give the chunks)."""
    from tensorsmith_hip import _lib

    b, h, s, d = LONG_B, LONG_H, LONG_S, D
    gen = torch.Generator(device="cuda").manual_seed(42)

    def draw(scale):
        return (torch.randn((b, h, s, d), generator=gen, device="cuda") * scale).to(torch.bfloat16)

    q, k, v = (ts.Tensor(draw(0.5), device="hip", requires_grad=True) for _ in range(3))
    upstream = ts.Tensor(draw(1.0), device="hip")

    def step():
        for t in (q, k, v):
            t.zero_grad()
        ts.nn.scaled_dot_product_attention(q, k, v, is_causal=True).backward(upstream)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    _lib.profile_reset()
    _lib.profile_enable(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.profile_enable(False)
    kernels = _lib.profile_read()
    flops = causal_fwd_flops(b, h, s, d) * 3.5
    ms = elapsed / steps * 1e3
    return {
        "ms_per_step": round(ms, 3),
        "value": round(flops / (ms * 1e-3) / 1e12, 1),
        "unit": "TFLOP/s",
        "frac": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "ds_chunks": kernels.get("bwd_dq_ds", (0, 0.0))[0] // max(steps, 1),
        "kernels": {n: {"launches": c, "mean_ms": round(t / max(c, 1), 4)} for n, (c, t) in kernels.items()},
        "config": {"workload": "causal_fwd_bwd_bf16_b16h16s8192d128", "batch": b, "heads": h,
                   "seq_len": s, "head_dim": d, "flop_per_step": flops},
    }


def bench_cached_step(ts, torch, steps, warmup):
    """One cached MultiHeadAttention decode step (E 4096, 32 query heads, 8 KV
    heads of 128, fp16, batch 64, 1024 cached positions): the q/k/v
    projections, RoPE and the K/V append in one kernel
    (tsattn_qkv_rope_append), then the decode kernel and the output
    projection -- against the same module with the fused kernel switched off
    (torch projections, then the RoPE-append kernel).  Random-init weights,
    synthetic activations."""
    from unittest.mock import patch

    import numpy as np

    from tensorsmith_hip import _lib, nn
    from tensorsmith_hip.nn.cache import KVCache

    bsz, embed, hq, hkv, cached = 64, 4096, 32, 8, 1024
    ts.seed(0)
    mha = nn.MultiHeadAttention(embed, hq, num_kv_heads=hkv, device="hip")
    mha.to(dtype="float16")
    mha.eval()
    cache = mha.new_cache(bsz, cached + 16, dtype="float16")
    rng = np.random.default_rng(0)
    x0 = ts.tensor((rng.standard_normal((bsz, cached, embed)) * 0.1).astype(np.float32), device="hip",
                   dtype="float16")
    x1 = ts.tensor((rng.standard_normal((bsz, 1, embed)) * 0.1).astype(np.float32), device="hip",
                   dtype="float16")
    with ts.no_grad():
        mha(x0, cache=cache)

    def step():
        with ts.no_grad():
            cache.truncate(cached)
            return mha(x1, cache=cache)

    out = {}
    for name, fn in (("fused", KVCache._project_append), ("unfused", lambda *a, **k: None)):
        with patch.object(KVCache, "_project_append", fn):
            for _ in range(warmup):
                step()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                step()
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) / steps * 1e3
            _lib.profile_reset()
            _lib.profile_enable(True)
            for _ in range(10):
                step()
            torch.cuda.synchronize()
            _lib.profile_enable(False)
            out[name] = {"ms_per_step": round(ms, 4),
                         "kernel_ms": {n: round(t / max(c, 1), 4) for n, (c, t) in _lib.profile_read().items()}}
    qkv_ms = out["fused"]["kernel_ms"]["qkv_rope_append"]
    # the algorithmic minimum: the weights once, x, the q and K/V rows
    qkv_bytes = float((hq + 2 * hkv) * 128 * embed * 2 + bsz * embed * 2 + bsz * (hq + 2 * hkv) * 128 * 2)
    out["qkv_rope_append"] = {
        "bytes_per_launch": qkv_bytes,
        "roofline": {"bound": "hbm", "achieved": round(qkv_bytes / (qkv_ms * 1e-3) / 1e9, 1),
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(qkv_bytes / (qkv_ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
                     "traffic": traffic_for("qkv_rope_append")}}
    out["config"] = {"workload": "mha_cached_step_f16_b64_e4096_h32kv8d128_len1024"}
    return out


def _bench_shapes(ts, torch, steps, warmup, shapes, dtype, path, peak):
    """Causal forward + backward through the public API at each (b, h, s, d)
    of `shapes` in `dtype` (N(0, 1) inputs); the kernel family `path` must
    run.  Per-kernel probe means and TFLOP/s against `peak`."""
    from tensorsmith_hip import _lib

    out = {}
    for name, (b, h, s, d) in shapes.items():
        gen = torch.Generator(device="cuda").manual_seed(7)
        raw = [torch.randn((b, h, s, d), generator=gen, device="cuda", dtype=torch.float32).to(dtype)
               for _ in range(4)]
        q, k, v = (ts.Tensor(t, device="hip", requires_grad=True) for t in raw[:3])
        upstream = ts.Tensor(raw[3], device="hip")

        def step():
            for t in (q, k, v):
                t.zero_grad()
            o = ts.nn.scaled_dot_product_attention(q, k, v, is_causal=True)
            o.backward(upstream)

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        if _lib.last_kernel_path() != path:
            raise RuntimeError(f"kernel family {_lib.last_kernel_path()} ran for {name}, expected {path}")
        _lib.profile_reset()
        _lib.profile_enable(True)
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / steps * 1e3
        _lib.profile_enable(False)
        kernels = {n: round(t / max(c, 1), 4) for n, (c, t) in _lib.profile_read().items()}
        tf = causal_fwd_flops(b, h, s, d) * 3.5 / (ms * 1e-3) / 1e12
        out[name] = {"ms_per_step": round(ms, 4), "tflops": round(tf, 2),
                     "frac_peak": round(tf / peak, 4), "kernel_ms": kernels}
    return out


def bench_fp32(ts, torch, steps, warmup):
    """Report-only: causal fp32 forward + backward through the public API (the
    path of fp32 models, the reference's default dtype) on the fp32 MFMA
    kernels: the reference's CPU-runnable case (B8 H4 S256 D64) and a long
    sequence (B2 H16 S2048 D128).  Fractions of the fp32 peak."""
    from tensorsmith_hip import _lib

    return _bench_shapes(ts, torch, steps, warmup,
                         {"causal_fwd_bwd_f32_b8h4s256d64": (8, 4, 256, 64),
                          "causal_fwd_bwd_f32_b2h16s2048d128": (2, 16, 2048, 128)},
                         torch.float32, _lib.PATH_MFMA, PEAK_FP32_TFLOPS)


def bench_head_dim32(ts, torch, steps, warmup):
    """Report-only: causal bf16 forward + backward at head dim 32 (the
    reference's default TransformerConfig, dim 128 over 4 heads) on the MFMA
    kernels: a small batch of its shape (B8 H4 S256) and B16 H16 S2048.
    Fractions of the bf16 peak."""
    from tensorsmith_hip import _lib

    return _bench_shapes(ts, torch, steps, warmup,
                         {"causal_fwd_bwd_bf16_b8h4s256d32": (8, 4, 256, 32),
                          "causal_fwd_bwd_bf16_b16h16s2048d32": (16, 16, 2048, 32)},
                         torch.bfloat16, _lib.PATH_MFMA, PEAK_BF16_TFLOPS)


def bench_lm(ts, torch, steps, warmup):
    """6-layer decoder LM, fp16 autocast, forward + backward, random init."""
    from tensorsmith_hip import _lib

    nn = ts.nn
    rng = torch.Generator(device="cuda").manual_seed(42)

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.ln1, self.ln2 = nn.LayerNorm(LM_DIM, device="hip"), nn.LayerNorm(LM_DIM, device="hip")
            self.attn = nn.MultiHeadAttention(LM_DIM, LM_HEADS, rotary=False, bias=True, device="hip")
            self.up = nn.Linear(LM_DIM, LM_FFN, device="hip")
            self.down = nn.Linear(LM_FFN, LM_DIM, device="hip")

        def forward(self, x):
            x = x + self.attn(self.ln1(x))
            return x + self.down(nn.functional.gelu(self.up(self.ln2(x))))

    class LM(nn.Module):
        def __init__(self):
            super().__init__()
            self.tok = nn.Embedding(LM_VOCAB, LM_DIM, device="hip")
            self.pos = nn.Embedding(LM_S, LM_DIM, device="hip")
            self.blocks = [Block() for _ in range(LM_LAYERS)]
            self.ln = nn.LayerNorm(LM_DIM, device="hip")
            self.head = nn.Linear(LM_DIM, LM_VOCAB, bias=False, device="hip")
            for name, prm in self.named_parameters():
                if not name.split(".")[-2].startswith("ln"):  # LayerNorm keeps gamma 1, beta 0
                    prm._data.normal_(0.0, 0.02, generator=rng)

        def forward(self, ids):
            b, s = ids.shape
            pos = ts.Tensor(torch.arange(s, device="cuda")[None].expand(b, s), device="hip")
            x = self.tok(ids) + self.pos(pos)
            for blk in self.blocks:
                x = blk(x)
            return self.head(self.ln(x))

    model = LM()
    ids = ts.Tensor(torch.randint(0, LM_VOCAB, (LM_B, LM_S), generator=rng, device="cuda"), device="hip")
    tgt = ts.Tensor(torch.randint(0, LM_VOCAB, (LM_B, LM_S), generator=rng, device="cuda"), device="hip")

    def step():
        for prm in model.parameters():
            prm.zero_grad()
        with ts.autocast("hip"):
            loss = nn.functional.cross_entropy(model(ids), tgt, axis=-1)
        loss.backward()
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    _lib.profile_reset()
    _lib.profile_enable(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.profile_enable(False)
    kernels = _lib.profile_read()
    ms = elapsed / steps * 1e3
    attn_ms = sum(t for n, (c, t) in kernels.items() if n in ATTN_KERNELS) / steps
    hd = LM_DIM // LM_HEADS
    attn_flops = causal_fwd_flops(LM_B, LM_HEADS, LM_S, hd) * 3.5 * LM_LAYERS
    tokens = LM_B * LM_S
    lin_flops = 6.0 * tokens * LM_LAYERS * (4 * LM_DIM * LM_DIM + 2 * LM_DIM * LM_FFN)
    head_flops = 6.0 * tokens * LM_DIM * LM_VOCAB
    return {
        "ms_per_step": ms,
        "value": tokens / (ms * 1e-3),
        "unit": "tokens/s",
        "loss": float(loss.item()),
        "attention_ms_per_step": attn_ms,
        "attention_share": attn_ms / ms,
        "flop_per_step": attn_flops + lin_flops + head_flops,
        "attention_flop_per_step": attn_flops,
        "kernels": {n: {"launches": c, "mean_ms": round(t / max(c, 1), 4)} for n, (c, t) in kernels.items()},
        "config": {"workload": "decoder_lm_6l_d512_h8_ffn2048_v32000_b8_s1024_fp16_autocast",
                   "layers": LM_LAYERS, "d_model": LM_DIM, "heads": LM_HEADS, "ffn": LM_FFN,
                   "vocab": LM_VOCAB, "batch": LM_B, "seq_len": LM_S},
    }


def cpu_threads():
    try:
        from threadpoolctl import threadpool_info

        counts = [i["num_threads"] for i in threadpool_info() if i.get("user_api") == "blas"]
        if counts:
            return max(counts)
    except Exception:  # noqa: BLE001 - reporting only
        pass
    return len(os.sched_getaffinity(0))


def cpu_host_info():
    """What the CPU leg ran on: the process's core affinity, the thread
    environment and the BLAS NumPy was built with."""
    import numpy as np

    info = {"affinity_cores": len(os.sched_getaffinity(0)),
            "OPENBLAS_NUM_THREADS": os.environ.get("OPENBLAS_NUM_THREADS"),
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}
    try:
        blas = np.show_config(mode="dicts")["Build Dependencies"]["blas"]
        info["blas"] = f"{blas.get('name')} {blas.get('version')}"
    except Exception:  # noqa: BLE001 - reporting only
        info["blas"] = None
    return info


def cpu_baseline(torch, host, dec_host, batches):
    """The NumPy oracle (reference algorithm) on a sample of the same inputs."""
    import numpy as np

    from oracle import attention as A

    def to_np(t):
        return t.float().cpu().numpy()

    # fwd+bwd: the first `batches` batch rows (all heads), streaming backend, block 64
    q, k, v, g = (to_np(host[x][:batches]) for x in ("q", "k", "v", "g"))

    def run():
        r = A.sdpa(q, k, v, None, True, dtype="bfloat16", backend="streaming", block_size=64)
        r.backward(g)

    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    flops = causal_fwd_flops(batches, H, S, D) * 3.5
    # decode: the reference's dense path on every sequence of the decode workload
    lens = dec_host["lengths"]
    nseq = DEC_B
    dq = to_np(dec_host["q"][:nseq])
    dk = [to_np(dec_host["k"][b, :, : lens[b]][None]) for b in range(nseq)]
    dv = [to_np(dec_host["v"][b, :, : lens[b]][None]) for b in range(nseq)]

    def dec():
        for b in range(nseq):
            A.sdpa(dq[b:b + 1], dk[b], dv[b], None, True, dtype="float16",
                   causal_offset=int(lens[b]) - 1, backend="dense")

    dec()
    dts = []
    for _ in range(5):
        t0 = time.perf_counter()
        dec()
        dts.append(time.perf_counter() - t0)
    dmed = float(np.median(dts))
    cores = cpu_threads()
    hinfo = cpu_host_info()
    return {
        "value": flops / med / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
        "host": hinfo,
        "sample": f"causal fwd+bwd of batch rows 0..{batches - 1} x {H} heads (S=2048 D=128, "
                  f"bf16 values in fp32), NumPy streaming block 64, median of 3: "
                  f"{med:.2f} s per sample",
        "decode": {"value": nseq / dmed, "unit": "tokens/s", "cores": cores, "kind": "port",
                   "host": hinfo,
                   "sample": f"dense decode of all {nseq} sequences (fp16 values in fp32), "
                             f"median of 5 after 1 warmup: {dmed:.3f} s"},
    }


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the attention path is per-GPU work with no collectives.", file=sys.stderr)
        sys.exit(2)
    import torch

    import tensorsmith_hip as ts

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (no GPU visible)", file=sys.stderr)
        sys.exit(2)
    if args.workload == "copy":
        # Calibration for rocprofv3 FETCH_SIZE / WRITE_SIZE: a device copy of
        # exactly 1 GiB (reads 1 GiB, writes 1 GiB), launched `steps` times.
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel() * 4, "launches": args.steps}), flush=True)
        return
    if args.workload == "decode":
        dec_res, _ = bench_decode(ts, torch, args.decode_steps, args.warmup)
        print(json.dumps({"decode": dec_res}), flush=True)
        return
    if args.workload == "decode_int8":
        _, dec_host = bench_decode(ts, torch, 2, 1)
        q8 = bench_decode_int8(ts, torch, args.decode_steps, args.warmup, dec_host)
        print(json.dumps({"decode_int8": q8}), flush=True)
        return
    if args.workload == "prefill":
        print(json.dumps({"prefill": bench_prefill(ts, torch, 3, 1)}), flush=True)
        return
    if args.workload == "lm":
        print(json.dumps({"lm_step": bench_lm(ts, torch, 5, 2)}), flush=True)
        return
    if args.workload == "cached_step":
        print(json.dumps({"cached_step": bench_cached_step(ts, torch, 50, 5)}), flush=True)
        return
    if args.workload == "long":
        print(json.dumps({"long_fwd_bwd": bench_long(ts, torch, 3, 1)}), flush=True)
        return
    if args.workload == "d32":
        print(json.dumps({"head_dim32": bench_head_dim32(ts, torch, 5, 2)}), flush=True)
        return
    if args.workload == "fp32":
        print(json.dumps({"fp32": bench_fp32(ts, torch, 5, 2)}), flush=True)
        return
    print(f"[bench] fwd+bwd B{B} H{H} S{S} D{D} bf16: {args.warmup} warmup + {args.steps} steps",
          file=sys.stderr, flush=True)
    main_res, host = bench_fwd_bwd(ts, torch, args.steps, args.warmup)
    print(f"[bench] fwd+bwd {main_res['ms_per_step']:.3f} ms/step", file=sys.stderr, flush=True)
    if args.workload == "fwd_bwd":
        print(json.dumps({"value": main_res["value"], "ms_per_step": main_res["ms_per_step"],
                          "step_ms": main_res["step_ms"],
                          "roofline": main_res["roofline"], "kernels": main_res["kernels"]}),
              flush=True)
        return
    if args.workload == "variants":
        print(json.dumps({"variants": bench_variants(ts, torch, args.steps, args.warmup, host)}),
              flush=True)
        return
    var_res = bench_variants(ts, torch, max(3, args.steps // 4), 2, host)
    print("[bench] variants " + ", ".join(f"{n} {r['ms_per_step']:.3f} ms" for n, r in var_res.items()),
          file=sys.stderr, flush=True)
    dec_res, dec_host = bench_decode(ts, torch, args.decode_steps, args.warmup)
    print(f"[bench] decode {dec_res['ms_per_step']:.3f} ms/step", file=sys.stderr, flush=True)
    q8_res = bench_decode_int8(ts, torch, args.decode_steps, args.warmup, dec_host)
    print(f"[bench] int8-cache decode {q8_res['ms_per_step']:.3f} ms/step", file=sys.stderr,
          flush=True)
    pf_res = bench_prefill(ts, torch, 3, 1)
    print(f"[bench] prefill {pf_res['ms_per_step']:.2f} ms/step", file=sys.stderr, flush=True)
    long_res = bench_long(ts, torch, 3, 1)
    print(f"[bench] fwd+bwd S8192 {long_res['ms_per_step']:.2f} ms/step ({long_res['ds_chunks']} dS chunks)",
          file=sys.stderr, flush=True)
    lm_res = bench_lm(ts, torch, 5, 2)
    print(f"[bench] lm step {lm_res['ms_per_step']:.2f} ms", file=sys.stderr, flush=True)
    cs_res = bench_cached_step(ts, torch, 50, 5)
    print(f"[bench] cached MHA step {cs_res['fused']['ms_per_step']:.3f} ms "
          f"(unfused {cs_res['unfused']['ms_per_step']:.3f} ms)", file=sys.stderr, flush=True)
    f32_res = bench_fp32(ts, torch, 5, 2)
    print("[bench] fp32 (fp32 MFMA kernels) " + ", ".join(
        f"{n} {r['ms_per_step']:.3f} ms" for n, r in f32_res.items()), file=sys.stderr, flush=True)
    d32_res = bench_head_dim32(ts, torch, 5, 2)
    print("[bench] bf16 head dim 32 " + ", ".join(
        f"{n} {r['ms_per_step']:.3f} ms" for n, r in d32_res.items()), file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu:
        print("[bench] cpu baseline (NumPy oracle sample)", file=sys.stderr, flush=True)
        cpu = cpu_baseline(torch, host, dec_host, args.cpu_batches)
        dec_res["cpu_baseline"] = cpu.pop("decode")
    line = {
        "metric": "attention fwd+bwd TFLOP/s at B16 H16 S2048 D128 bf16; decode tokens/s",
        "value": round(main_res["value"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_res["ms_per_step"], 4),
        "step_ms": main_res["step_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*0.5 q/k/v, N(0,1) dO, generated on device)",
        "config": {"workload": "causal_fwd_bwd_bf16_b16h16s2048d128", "batch": B, "heads": H,
                   "seq_len": S, "head_dim": D, "causal": True,
                   "flop_per_step": causal_fwd_flops(B, H, S, D) * 3.5},
        "roofline": main_res["roofline"],
        # the whole step (forward + backward, algorithmic FLOP / step time)
        "step_roofline": {"bound": "mfma", "achieved": round(main_res["value"], 1),
                          "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                          "frac": round(main_res["value"] / PEAK_BF16_TFLOPS, 4)},
        "kernels": main_res["kernels"],
        "variants": var_res,
        "cpu_baseline": cpu,
        "decode": dec_res,
        "decode_int8": q8_res,
        "prefill": pf_res,
        "long_fwd_bwd": long_res,
        "lm_step": lm_res,
        "cached_step": cs_res,
        "fp32": f32_res,
        "head_dim32": d32_res,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
