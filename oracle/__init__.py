"""CPU oracle for nlearn's hot path — TEST INFRASTRUCTURE ONLY.

A float64 NumPy restatement of the reference algorithms (causal attention
forward/backward, bf16 GEMM with fp32-or-better accumulation, softmax
cross-entropy, the training step). Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker or the reported CPU baseline. The product path (``nlearn_amd``) never
imports it and has no CPU fallback.

Pinning status of each function (how it is checked, beyond its own formula):
  bf16_round ........ pinned: bit-exact vs torch.bfloat16 casts (RNE, NaN, inf)
  gemm .............. pinned: exact small-integer products, transpose identities,
                      float64 NumPy matmul
  flash_fwd ......... pinned: torch float64 materialised attention, row-0 and
                      equal-key closed forms, NaN-poisoned future keys
  flash_bwd ......... pinned: torch float64 autograd, finite differences,
                      sum(dV) = sum(dO), sum(dK) = 0
  ce ................ pinned: torch float64 cross_entropy + autograd, uniform
                      logits -> ln V, sum(dlogits) = 0 per row
  model step ........ pinned: torch float64 autograd of the same network,
                      finite differences, AdamW closed form on a scalar
There are no stored reference outputs to compare against (the reference's
tests recompute their references live); the JAX/XLA-CPU numerics of the
reference's pure-JAX path are therefore not bit-pinned.
"""
