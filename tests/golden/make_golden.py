"""Write the attention golden fixtures (``attention_golden.npz``).

The reference ships no golden vectors (its tests regenerate inputs from
seeds), so these fixtures are computed by an independent library:
``torch.nn.functional.scaled_dot_product_attention`` and autograd in float64
on the CPU.  Cases follow the shapes and seeds of the reference's own tests
in ``tests/test_transformer.py``:

* ``vjp_offset``   -- ``:40-54``  Sq=3, Sk=5, Dqk=4, Dv=3, causal_offset=2
* ``masked``       -- ``:56-92``  bool mask with a fully masked row, causal
* ``gqa``          -- ``:94-119`` 4 query heads over 2 KV heads
* ``unmasked_*``   -- ``:127-140`` causal / non-causal, [1,2,7,8]
* ``float_mask``   -- additive float mask with ``-inf`` and finite entries
* ``ragged``       -- Sq=70, Sk=133, key padding + offset (odd tiles)

Fully masked rows follow the reference contract (output 0, gradients 0,
LSE ``-inf``; ``src/tensorsmith/nn/attention.py:126-127,194-196``): torch
would return NaN there, so those rows are zeroed and their upstream gradient
is zero in the torch graph, which leaves every other gradient unchanged.

Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).with_name("attention_golden.npz")


def allowed(b, h, sq, sk, mask, causal, offset):
    a = np.ones((b, h, sq, sk), bool)
    if mask is not None:
        m = np.broadcast_to(mask, (b, h, sq, sk))
        a &= m if m.dtype == np.bool_ else np.isfinite(m)
    if causal:
        a &= (np.arange(sq)[:, None] + offset) >= np.arange(sk)[None, :]
    return a


def case(q, k, v, g, mask=None, causal=False, offset=0, scale=None, gqa=False):
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    rep = hq // hkv
    mult = 1 / math.sqrt(d) if scale is None else scale
    ok = allowed(b, hq, sq, sk, mask, causal, offset)
    live = ok.any(-1)  # [b,h,sq]
    tq, tk, tv = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    ek = tk.repeat_interleave(rep, dim=1) if rep > 1 else tk
    ev = tv.repeat_interleave(rep, dim=1) if rep > 1 else tv
    # additive float mask: finite entries add, -inf removes; bool: True keeps
    bias = np.zeros((b, hq, sq, sk))
    if mask is not None and np.asarray(mask).dtype != np.bool_:
        bias = np.where(np.isfinite(np.broadcast_to(mask, bias.shape)),
                        np.broadcast_to(mask, bias.shape), 0.0)
    keep = ok.copy()
    keep[~live] = True  # dummy keys for dead rows (zeroed below)
    tbias = torch.tensor(np.where(keep, bias, -np.inf))
    out = torch.nn.functional.scaled_dot_product_attention(tq, ek, ev, attn_mask=tbias, scale=mult)
    tg = torch.tensor(np.where(live[..., None], g, 0.0))
    (out * tg).sum().backward()
    s = (tq.detach() @ ek.detach().transpose(-1, -2)) * mult + torch.tensor(bias)
    s = s.masked_fill(~torch.tensor(ok), -math.inf)
    lse = torch.logsumexp(s, dim=-1).numpy()
    o = np.where(live[..., None], out.detach().numpy(), 0.0)
    return {
        "q": q, "k": k, "v": v, "g": g, "out": o, "lse": np.where(live, lse, -np.inf),
        "dq": tq.grad.numpy(), "dk": tk.grad.numpy(), "dv": tv.grad.numpy(),
        "mask": np.zeros(0) if mask is None else np.asarray(mask),
        "meta": np.array([int(causal), offset, 0 if scale is None else 1,
                          mult, int(gqa)], dtype=np.float64),
    }


def main():
    cases = {}
    np.random.seed(19)  # the reference tests' seed (tests/test_transformer.py:37-38)
    q, k, v = np.random.randn(1, 2, 3, 4), np.random.randn(1, 2, 5, 4), np.random.randn(1, 2, 5, 3)
    cases["vjp_offset"] = case(q, k, v, np.random.randn(1, 2, 3, 3), causal=True, offset=2)
    raw = [np.random.randn(2, 2, 4, 4) for _ in range(3)]
    boolean = np.ones((4, 4), dtype=bool)
    boolean[1] = False
    boolean[3, 0] = False
    cases["masked"] = case(*raw, np.random.randn(2, 2, 4, 4), mask=boolean, causal=True)
    q, k, v = np.random.randn(1, 4, 3, 4), np.random.randn(1, 2, 5, 4), np.random.randn(1, 2, 5, 4)
    cases["gqa"] = case(q, k, v, np.random.randn(1, 4, 3, 4), gqa=True)
    raw = [np.random.randn(1, 2, 7, 8) for _ in range(3)]
    g = np.random.randn(1, 2, 7, 8)
    cases["unmasked_causal"] = case(*raw, g, causal=True)
    cases["unmasked_full"] = case(*raw, g, causal=False)
    rng = np.random.default_rng(7)
    raw = [rng.standard_normal((2, 3, 6, 16)) for _ in range(3)]
    fmask = rng.standard_normal((1, 1, 6, 6))
    fmask[0, 0, 2, :] = -np.inf  # a fully masked row
    fmask[0, 0, 4, 1] = -np.inf
    cases["float_mask"] = case(*raw, rng.standard_normal((2, 3, 6, 16)), mask=fmask, scale=0.3)
    q = rng.standard_normal((2, 2, 70, 16))
    k = rng.standard_normal((2, 2, 133, 16))
    v = rng.standard_normal((2, 2, 133, 16))
    lengths = np.array([133, 101])
    kp = (np.arange(133)[None, :] < lengths[:, None])[:, None, None, :]
    cases["ragged"] = case(q, k, v, rng.standard_normal((2, 2, 70, 16)), mask=kp,
                           causal=True, offset=63)
    flat = {f"{name}/{key}": val for name, c in cases.items() for key, val in c.items()}
    np.savez_compressed(OUT, **flat)
    print(f"wrote {OUT} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
