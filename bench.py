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
* ``decode`` -- KV-cache decode (B=64 H=32 D=128 fp16 cache, lengths
  U[512, 8192]): tokens/s and HBM GB/s with its own roofline;
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
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "custom-ml-library_amd"))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E
B, H, S, D = 16, 16, 2048, 128
DEC_B, DEC_H, DEC_D, DEC_CAP, DEC_LO, DEC_HI = 64, 32, 128, 8192, 512, 8192


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
    ap.add_argument("--workload", choices=["all", "fwd_bwd", "decode", "copy"], default="all",
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
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.profile_enable(False)
    kernels = _lib.profile_read()
    fwd = causal_fwd_flops(B, H, S, D)
    flops = fwd * 3.5
    ms = elapsed / steps * 1e3
    # algorithmic FLOP per launch: forward kernel = QK^T + PV (2 GEMMs);
    # dK/dV kernel = S recompute, dP, dV, dK (4 of the backward's 5 GEMMs);
    # dQ kernel = dQ (1 GEMM; its S/dP recompute is overhead, not counted)
    work = {"fwd_mfma": fwd, "bwd_dkdv_mfma": 2.0 * fwd, "bwd_dq_mfma": 0.5 * fwd}
    per_kernel = {n: {"launches": c, "mean_ms": t / max(c, 1)} for n, (c, t) in kernels.items()}
    dom = max((n for n in per_kernel if n in work), key=lambda n: per_kernel[n]["mean_ms"])
    achieved = work[dom] / (per_kernel[dom]["mean_ms"] * 1e-3) / 1e12
    for n, w in work.items():
        if n in per_kernel:
            per_kernel[n]["tflops"] = round(w / (per_kernel[n]["mean_ms"] * 1e-3) / 1e12, 1)
    result = {
        "ms_per_step": ms,
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


def cpu_threads():
    try:
        from threadpoolctl import threadpool_info

        counts = [i["num_threads"] for i in threadpool_info() if i.get("user_api") == "blas"]
        if counts:
            return max(counts)
    except Exception:  # noqa: BLE001 - reporting only
        pass
    return len(os.sched_getaffinity(0))


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
    return {
        "value": flops / med / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
        "sample": f"causal fwd+bwd of batch rows 0..{batches - 1} x {H} heads (S=2048 D=128, "
                  f"bf16 values in fp32), NumPy streaming block 64, median of 3: "
                  f"{med:.2f} s per sample",
        "decode": {"value": nseq / dmed, "unit": "tokens/s", "cores": cores, "kind": "port",
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
    print(f"[bench] fwd+bwd B{B} H{H} S{S} D{D} bf16: {args.warmup} warmup + {args.steps} steps",
          file=sys.stderr, flush=True)
    main_res, host = bench_fwd_bwd(ts, torch, args.steps, args.warmup)
    print(f"[bench] fwd+bwd {main_res['ms_per_step']:.3f} ms/step", file=sys.stderr, flush=True)
    if args.workload == "fwd_bwd":
        print(json.dumps({"value": main_res["value"], "ms_per_step": main_res["ms_per_step"],
                          "roofline": main_res["roofline"], "kernels": main_res["kernels"]}),
              flush=True)
        return
    dec_res, dec_host = bench_decode(ts, torch, args.decode_steps, args.warmup)
    print(f"[bench] decode {dec_res['ms_per_step']:.3f} ms/step", file=sys.stderr, flush=True)
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
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*0.5 q/k/v, N(0,1) dO, generated on device)",
        "config": {"workload": "causal_fwd_bwd_bf16_b16h16s2048d128", "batch": B, "heads": H,
                   "seq_len": S, "head_dim": D, "causal": True,
                   "flop_per_step": causal_fwd_flops(B, H, S, D) * 3.5},
        "roofline": main_res["roofline"],
        "kernels": main_res["kernels"],
        "cpu_baseline": cpu,
        "decode": dec_res,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
