"""CPU oracle for the attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, the reference's attention algorithm
(tensorsmith ``src/tensorsmith/nn/attention.py:16-252`` and the KV-cache
quantiser ``src/tensorsmith/nn/cache.py:54-99``).  It exists to check the HIP
kernels, never to stand in for them:

* only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
  ``bench.py`` may import it;
* the product package (``custom-ml-library_amd/tensorsmith_hip``) never
  imports it and has no CPU fallback.

How each function is pinned (tests live in ``tests/test_oracle.py``):

* forward values: float64 brute force, ``torch.nn.functional.
  scaled_dot_product_attention`` in float64 on the CPU, and the committed
  golden fixtures under ``tests/golden/`` (written by torch, not by this
  package);
* online-softmax equivalence: streaming == dense for every block size;
* VJP: torch autograd in float64, float64 central differences (the method of
  the reference's ``tests/test_transformer.py:13-33``), and the invariant
  ``sum_j dS_ij == 0``;
* masks / causal offset / fully-masked rows: explicit-mask brute force and
  the zero-row contract;
* GQA: equality with MHA on ``repeat_interleave``-expanded K/V;
* bf16 / fp16 rounding: ``torch.Tensor.to(bfloat16 / float16)``;
* int8 KV quantisation: closed form and the half-step error bound.

No function here is "parity unpinned".
"""
