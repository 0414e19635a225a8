"""Write the small golden fixtures under tests/golden/ from the float64 oracle.

The reference stores no golden vectors (its checks recompute NumPy references
live); these fixtures freeze the oracle's outputs for the reference's own
seeds and shapes so GPU tests need no recomputation:
  flash:  seed 1, (2,128,64)  validate_flash_tiled.py:12-17
          seed 2, (2,128,64)  validate_flash_bwd128.py:9-15 (with dO)
  gemm:   default_rng(0), (64,128,64) x0.1 / (256,512,256) x1 / (64,128,64) x300
          check_gemm_bf16.py:12-28
  ce:     default_rng(0), (512,1024) N(0,1)   check_ce.py:15-19
          (dlogits stored for the first 64 rows only, to keep the file small)
Inputs are stored as bf16 bit patterns (what the kernels consume); expected
outputs are computed in float64 on those bf16 values and stored as float32.
Run: python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from oracle import ops  # noqa: E402


def _f32(**arrs):
    return {k: np.asarray(v, np.float32) for k, v in arrs.items()}


def flash_case(seed, shape, name):
    np.random.seed(seed)
    Q = np.random.randn(*shape).astype(np.float32)
    K = np.random.randn(*shape).astype(np.float32)
    V = np.random.randn(*shape).astype(np.float32)
    dO = np.random.randn(*shape).astype(np.float32)
    qb, kb, vb, db = (ops.bf16_bits(a) for a in (Q, K, V, dO))
    q, k, v, d = (ops.bf16_to_f32(a) for a in (qb, kb, vb, db))
    O, L = ops.flash_fwd(q, k, v)
    dQ, dK, dV, D = ops.flash_bwd(q, k, v, d)
    np.savez_compressed(HERE / f"{name}.npz", Q=qb, K=kb, V=vb, dO=db, **_f32(O=O, L=L, dQ=dQ, dK=dK, dV=dV, D=D))


def gemm_case(M, K, N, scale, name):
    rng = np.random.default_rng(0)
    A = (rng.standard_normal((M, K)) * scale).astype(np.float32)
    B = (rng.standard_normal((K, N)) * scale).astype(np.float32)
    ab, bb = ops.bf16_bits(A), ops.bf16_bits(B)
    C = ops.gemm(ops.bf16_to_f32(ab), ops.bf16_to_f32(bb))
    np.savez_compressed(HERE / f"{name}.npz", A=ab, B=bb, **_f32(C=C))


def ce_case(M, V, name):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((M, V)).astype(np.float32)
    t = rng.integers(0, V, (M,)).astype(np.int32)
    xb = ops.bf16_bits(x)
    loss, lse, dl = ops.ce(ops.bf16_to_f32(xb), t)
    np.savez_compressed(HERE / f"{name}.npz", logits=xb, targets=t, **_f32(loss=loss, lse=lse, dlogits_head=dl[:64]))


if __name__ == "__main__":
    flash_case(1, (2, 128, 64), "flash_s1_2x128x64")
    flash_case(2, (2, 128, 64), "flash_s2_2x128x64")
    gemm_case(64, 128, 64, 0.1, "gemm_small")
    gemm_case(256, 512, 256, 1.0, "gemm_medium")
    gemm_case(64, 128, 64, 300.0, "gemm_large_magnitude")
    ce_case(512, 1024, "ce_512x1024")
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))
