"""Float64 NumPy restatement of the three hot-path ops. TEST INFRASTRUCTURE ONLY.

Each function cites the reference lines it restates (paths relative to the
nlearn repository).
"""
from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# bfloat16
# ---------------------------------------------------------------------------


def bf16_bits(x) -> np.ndarray:
    """float -> bfloat16 bit patterns (uint16), round-to-nearest-even; NaN -> quiet NaN.

    The reference casts operands to bf16 before its kernels (gemm.py:51-52,
    model.py:372-375); this is that cast.
    """
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32)
    # finite values cannot overflow 32 bits here (largest is 0xFF7FFFFF + 0x8000);
    # NaN patterns are replaced below
    r = u >> 16                       # (u + 0x7FFF + lsb) >> 16, in place on one temporary
    r &= np.uint32(1)
    r += np.uint32(0x7FFF)
    r += u
    r >>= 16
    r = r.astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        r = np.where(nan, ((u >> 16) | np.uint32(0x40)).astype(np.uint16), r)
    return r


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x) -> np.ndarray:
    """Round to bf16 and back to float32."""
    return bf16_to_f32(bf16_bits(x))


# ---------------------------------------------------------------------------
# GEMM — gemm.py:43-79, gemm.metal:48-115
# ---------------------------------------------------------------------------


def gemm(A, B, opA: str = "N", opB: str = "N") -> np.ndarray:
    """op(A) @ op(B) in float64 on bf16-rounded operands.

    opA = "T" means A is stored [K, M] and used transposed (dB = A^T dC,
    gemm.py:75); opB = "T" means B is stored [N, K] (dA = dC B^T, gemm.py:74).
    """
    a = bf16_round(A).astype(np.float64)
    b = bf16_round(B).astype(np.float64)
    if opA == "T":
        a = a.T
    if opB == "T":
        b = b.T
    return a @ b


# ---------------------------------------------------------------------------
# causal attention — attention.py:138-156 (forward), flash_attention.metal:55-146
# (L = max + log sum exp), validate_flash_bwd.py:31-38 (analytic backward)
# ---------------------------------------------------------------------------


def _scale(d: int, scale):
    return 1.0 / np.sqrt(d) if scale is None else float(scale)


def flash_fwd(Q, K, V, scale=None, causal: bool = True):
    """O = softmax(scale Q K^T + mask) V and L = logsumexp of each score row.

    Q, K, V: (n, s, d). Returns O (n, s, d) and L (n, s), float64.
    """
    Q = np.asarray(Q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    n, s, d = Q.shape
    sc = _scale(d, scale)
    S = np.einsum("nqd,nkd->nqk", Q, K) * sc
    if causal:
        mask = np.triu(np.ones((s, s), bool), 1)
        S = np.where(mask[None], -np.inf, S)
    m = S.max(-1, keepdims=True)
    e = np.exp(S - m)
    l = e.sum(-1, keepdims=True)
    P = e / l
    O = np.einsum("nqk,nkd->nqd", P, V)
    L = (m + np.log(l))[..., 0]
    return O, L


def flash_bwd(Q, K, V, dO, scale=None, causal: bool = True):
    """dQ, dK, dV of sum(O * dO) with P recomputed from L, plus D = rowsum(dO * O).

    dV = P^T dO; dP = dO V^T; dS = P (dP - D); dQ = scale dS K; dK = scale dS^T Q
    (validate_flash_bwd.py:31-38; D as attention.py:116).
    """
    Q = np.asarray(Q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    dO = np.asarray(dO, np.float64)
    n, s, d = Q.shape
    sc = _scale(d, scale)
    O, L = flash_fwd(Q, K, V, sc, causal)
    S = np.einsum("nqd,nkd->nqk", Q, K) * sc
    P = np.exp(S - L[..., None])
    if causal:
        P = np.where(np.triu(np.ones((s, s), bool), 1)[None], 0.0, P)
    D = np.einsum("nqd,nqd->nq", dO, O)
    dV = np.einsum("nqk,nqd->nkd", P, dO)
    dP = np.einsum("nqd,nkd->nqk", dO, V)
    dS = P * (dP - D[..., None])
    dQ = np.einsum("nqk,nkd->nqd", dS, K) * sc
    dK = np.einsum("nqk,nqd->nkd", dS, Q) * sc
    return dQ, dK, dV, D


# ---------------------------------------------------------------------------
# cross-entropy — cross_entropy.py:49-81, cross_entropy.metal:38-97
# ---------------------------------------------------------------------------


def ce(logits, targets, scale=None):
    """Per-row loss, lse and dlogits = (softmax - onehot) * scale (default 1/M)."""
    x = np.asarray(logits, np.float64)
    t = np.asarray(targets, np.int64)
    M, V = x.shape
    m = x.max(-1, keepdims=True)
    lse = (m + np.log(np.exp(x - m).sum(-1, keepdims=True)))[:, 0]
    loss = lse - x[np.arange(M), t]
    sc = (1.0 / M) if scale is None else float(scale)
    dl = np.exp(x - lse[:, None])
    dl[np.arange(M), t] -= 1.0
    return loss, lse, dl * sc


# ---------------------------------------------------------------------------
# fused LM head + cross-entropy — cross_entropy.py:84-170
# ---------------------------------------------------------------------------


def linear_ce(X, W, targets, chunk: int = 4096, round_bf16: bool = True):
    """linear_cross_entropy with g = 1: (loss, lse, dX, dW).

    Follows the reference's chunked form: the forward folds each vocabulary
    chunk's logits into an online (max, sum) and keeps the target's logit
    (cross_entropy.py:102-116); the backward recomputes each chunk's logits and
    accumulates dX and the chunk's dW columns (cross_entropy.py:133-161). With
    ``round_bf16`` the logits and dlogits are rounded to bf16 before use, as the
    reference's bf16 matmul outputs and operands are (gemm.py:51-52, 115).
    """
    X = np.asarray(X, np.float64)
    W = np.asarray(W, np.float64)
    t = np.asarray(targets, np.int64)
    M, D = X.shape
    V = W.shape[1]
    rows = np.arange(M)
    rnd = (lambda a: bf16_round(a).astype(np.float64)) if round_bf16 else (lambda a: a)
    run_max = np.full(M, -np.inf)
    run_sum = np.zeros(M)
    correct = np.zeros(M)
    for cs in range(0, V, chunk):
        lc = rnd(X @ W[:, cs:cs + chunk])
        nm = np.maximum(run_max, lc.max(-1))
        run_sum = run_sum * np.exp(run_max - nm) + np.exp(lc - nm[:, None]).sum(-1)
        run_max = nm
        inc = (t >= cs) & (t < cs + lc.shape[1])
        correct[inc] = lc[rows[inc], t[inc] - cs]
    lse = run_max + np.log(run_sum)
    loss = float((lse - correct).mean())
    dX = np.zeros((M, D))
    dW = np.zeros((D, V))
    for cs in range(0, V, chunk):
        Wc = W[:, cs:cs + chunk]
        lc = rnd(X @ Wc)
        dl = np.exp(lc - lse[:, None])
        inc = (t >= cs) & (t < cs + lc.shape[1])
        dl[rows[inc], t[inc] - cs] -= 1.0
        dl = rnd(dl / M)
        dX += dl @ Wc.T
        dW[:, cs:cs + chunk] = X.T @ dl
    return loss, lse, dX, dW
