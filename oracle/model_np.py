"""NumPy restatement of the BASELINE training step — TEST INFRASTRUCTURE ONLY.

Forward, hand-written backward and AdamW of the GPT-style decoder the build
trains (d_model 512, 8 heads, 4 layers, FFN 2048 tanh-GELU with biases,
pre-LayerNorm, learned positions, untied LM head, vocab 50257), following:

  nlearn/train.py:270-285     batch loss: CE of predicting batch[:, 1:] from batch[:, :-1]
  nlearn/train.py:487-505     optax.adamw + warmup_cosine_decay_schedule
  nlearn/attention.py:138-156 causal softmax attention, scale 1/sqrt(d_head)
  nlearn/kernels/gemm.py:93-115 linear = x @ W on bf16 operands
  nlearn/model.py:361-398     embed -> blocks -> final LayerNorm -> LM head

Arithmetic is float32 with operands rounded to bf16 where the device path
computes in bf16 (weights, GEMM inputs), so the two paths agree to bf16
accumulation noise. Parameters use the same nested-dict layout as
nlearn_amd.model (W_q|W_k|W_v stored as one [d, 3d] matrix).

Pinned by: tests/test_model_oracle.py (float64 torch autograd of the same
network on a small configuration, AdamW and schedule closed forms).
"""
from __future__ import annotations

import concurrent.futures as cf_threads
import math
import os

import numpy as np

from .ops import bf16_round as _bf16

GELU_C = math.sqrt(2.0 / math.pi)


class Config:
    def __init__(self, vocab=50257, d=512, heads=8, layers=4, ff=2048, max_seq=512, eps=1e-5):
        self.vocab, self.d, self.heads, self.layers, self.ff, self.max_seq, self.eps = (
            vocab, d, heads, layers, ff, max_seq, eps)


BASELINE = Config()


def init_params(seed=0, cfg: Config = BASELINE):
    """Same draws as nlearn_amd.model.init_params_numpy (N(0,0.02) weights,
    gamma 1, beta/bias 0) in the same order."""
    rng = np.random.default_rng(seed)
    d, f = cfg.d, cfg.ff

    def w(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).astype(np.float32)

    p = {"embeddings": {"token_embed": w(cfg.vocab, d), "pos_embed": w(cfg.max_seq, d)}, "blocks": []}
    for _ in range(cfg.layers):
        p["blocks"].append({
            "ln1": {"gamma": np.ones(d, np.float32), "beta": np.zeros(d, np.float32)},
            "attn": {"W_qkv": w(d, 3 * d), "W_o": w(d, d)},
            "ln2": {"gamma": np.ones(d, np.float32), "beta": np.zeros(d, np.float32)},
            "ffn": {"W1": w(d, f), "b1": np.zeros(f, np.float32), "W2": w(f, d), "b2": np.zeros(d, np.float32)},
        })
    p["ln_final"] = {"gamma": np.ones(d, np.float32), "beta": np.zeros(d, np.float32)}
    p["lm_head"] = w(d, cfg.vocab)
    return p


def _map(fn, tree):
    if isinstance(tree, dict):
        return {k: _map(fn, v) for k, v in tree.items()}
    if isinstance(tree, list):
        return [_map(fn, v) for v in tree]
    return fn(tree)


def _leaves(tree):
    if isinstance(tree, dict):
        return [x for k in tree for x in _leaves(tree[k])]
    if isinstance(tree, list):
        return [x for v in tree for x in _leaves(v)]
    return [tree]


def _ident(a):
    return a


def _ln_fwd(x, g, b, eps):
    mu = x.mean(-1, keepdims=True)
    xc = x - mu
    var = (xc * xc).mean(-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    xh = xc * rstd
    return xh * g + b, (xh, rstd)


def _ln_bwd(dy, g, cache):
    xh, rstd = cache
    dxh = dy * g
    n = xh.shape[-1]
    dx = rstd / n * (n * dxh - dxh.sum(-1, keepdims=True) - xh * (dxh * xh).sum(-1, keepdims=True))
    dg = (dy * xh).reshape(-1, n).sum(0)
    db = dy.reshape(-1, n).sum(0)
    return dx, dg, db


def _gelu(u):
    t = np.tanh(GELU_C * (u + 0.044715 * (u * u * u)))
    return 0.5 * u * (1.0 + t), t


def _gelu_bwd(du_out, u, t):
    dt = (1.0 - t * t) * GELU_C * (1.0 + 3 * 0.044715 * u * u)
    return du_out * (0.5 * (1.0 + t) + 0.5 * u * dt)


def _per_head(fn, bs: int, H: int) -> None:
    """fn(b, h) for every head, on a thread pool (NumPy releases the GIL in
    its array loops, so long sequences use every host core)."""
    with cf_threads.ThreadPoolExecutor(max_workers=max(1, min(16, len(os.sched_getaffinity(0))))) as ex:
        list(ex.map(lambda bh: fn(*bh), [(b, h) for b in range(bs) for h in range(H)]))


def _attention_fwd(q, k, v, scale, mask):
    """Materialised causal attention (attention.py:138-156), one head at a time:
    P = softmax(scale * q k^T with the future masked to -inf), O = P v.
    q, k, v: (bs, H, S, dh). Returns O and P (kept for the backward)."""
    bs, H, S, _ = q.shape
    o = np.empty_like(q)
    pr = np.empty((bs, H, S, S), dtype=q.dtype)

    def head(b, h):
        s = (q[b, h] @ k[b, h].T) * scale
        s[mask] = -np.inf
        s -= s.max(-1, keepdims=True)
        p = np.exp(s, out=s)
        p /= p.sum(-1, keepdims=True)
        pr[b, h] = p
        o[b, h] = p @ v[b, h]

    _per_head(head, bs, H)
    return o, pr


def _attention_bwd(q, k, v, pr, do, scale):
    """Analytic backward of _attention_fwd (validate_flash_bwd.py:31-38):
    dV = P^T dO, dP = dO V^T, dS = P (dP - rowsum(dP P)), dQ = scale dS K,
    dK = scale dS^T Q; one head at a time."""
    bs, H = q.shape[:2]
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)

    def head(b, h):
        p = pr[b, h]
        dv[b, h] = p.T @ do[b, h]
        dp = do[b, h] @ v[b, h].T
        ds = p * (dp - (dp * p).sum(-1, keepdims=True))
        dq[b, h] = (ds @ k[b, h]) * scale
        dk[b, h] = (ds.T @ q[b, h]) * scale

    _per_head(head, bs, H)
    return dq, dk, dv


def loss_and_grads(params, batch, cfg: Config = BASELINE, exact: bool = False, grads: bool = True):
    """Mean next-token CE of a (bs, seq+1) batch and the gradient of every parameter.

    exact=True drops every bf16 rounding (pure float arithmetic of the input
    dtype), which is what the float64 autograd cross-check compares against.
    grads=False returns (loss, None) after the forward.
    """
    bf16_round = _ident if exact else _bf16

    def _mm(a, b):  # GEMM on bf16-rounded operands, fp32 result (gemm.py:51-52)
        return bf16_round(a) @ bf16_round(b)

    ids, tg = batch[:, :-1], batch[:, 1:]
    bs, S = ids.shape
    d, H = cfg.d, cfg.heads
    dh = d // H
    scale = 1.0 / math.sqrt(dh)
    P = params
    E, Pe = P["embeddings"]["token_embed"], P["embeddings"]["pos_embed"]
    x = bf16_round(E[ids] + Pe[:S][None])
    caches = []
    mask = np.triu(np.ones((S, S), bool), 1)
    for blk in P["blocks"]:
        c = {}
        h, c["ln1"] = _ln_fwd(x, blk["ln1"]["gamma"], blk["ln1"]["beta"], cfg.eps)
        h = bf16_round(h)
        qkv = bf16_round(_mm(h.reshape(-1, d), blk["attn"]["W_qkv"])).reshape(bs, S, 3, H, dh)
        q, k, v = (np.ascontiguousarray(qkv[:, :, i].transpose(0, 2, 1, 3)) for i in range(3))
        o, pr = _attention_fwd(q, k, v, scale, mask)
        a = bf16_round(o.transpose(0, 2, 1, 3).reshape(bs, S, d))
        x1 = bf16_round(x + bf16_round(_mm(a.reshape(-1, d), blk["attn"]["W_o"])).reshape(bs, S, d))
        h2, c["ln2"] = _ln_fwd(x1, blk["ln2"]["gamma"], blk["ln2"]["beta"], cfg.eps)
        h2 = bf16_round(h2)
        u = _mm(h2.reshape(-1, d), blk["ffn"]["W1"]) + blk["ffn"]["b1"]
        gu, t = _gelu(bf16_round(u))
        gu = bf16_round(gu)
        y = bf16_round(_mm(gu, blk["ffn"]["W2"]) + blk["ffn"]["b2"])
        x2 = bf16_round(x1 + y.reshape(bs, S, d))
        c.update(h=h, q=q, k=k, v=v, pr=pr, a=a, h2=h2, u=bf16_round(u), t=t, gu=gu)
        caches.append(c)
        x = x2
    hf, cf = _ln_fwd(x, P["ln_final"]["gamma"], P["ln_final"]["beta"], cfg.eps)
    hf = bf16_round(hf)
    # LM head + CE and their backward, in blocks of rows (the (M, V) logits of
    # one block at a time; blocks run on a thread pool, NumPy releases the GIL)
    hf2 = bf16_round(hf.reshape(-1, d))
    Wb = bf16_round(P["lm_head"])
    M = hf2.shape[0]
    t_flat = tg.reshape(-1)

    def head_block(r0, r1):
        logits = bf16_round(hf2[r0:r1] @ Wb)                               # (rows, V)
        rows = np.arange(r1 - r0)
        tb = t_flat[r0:r1]
        mx = logits.max(-1, keepdims=True)
        lse = (mx + np.log(np.exp(logits - mx).sum(-1, keepdims=True)))[:, 0]
        loss_rows = lse - logits[rows, tb]
        if not grads:
            return loss_rows, None, None
        dl = np.exp(logits - lse[:, None])                                  # softmax
        dl[rows, tb] -= 1.0
        dl = bf16_round(dl / M)
        return loss_rows, dl @ Wb.T, hf2[r0:r1].T @ dl

    blk = 1024
    starts = list(range(0, M, blk))
    with cf_threads.ThreadPoolExecutor(max_workers=max(1, min(16, len(os.sched_getaffinity(0))))) as ex:
        parts = list(ex.map(lambda r0: head_block(r0, min(r0 + blk, M)), starts))
    loss = float(np.concatenate([p[0] for p in parts]).mean())
    if not grads:
        return loss, None

    # ---- backward ----
    G = _map(np.zeros_like, P)
    G["lm_head"] = parts[0][2].copy()
    for p in parts[1:]:                                                     # fixed order
        G["lm_head"] += p[2]
    dhf = np.concatenate([p[1] for p in parts]).reshape(bs, S, d)
    del parts
    dx, G["ln_final"]["gamma"], G["ln_final"]["beta"] = _ln_bwd(dhf, P["ln_final"]["gamma"], cf)
    for li in range(cfg.layers - 1, -1, -1):
        blk, c, gb = P["blocks"][li], caches[li], G["blocks"][li]
        # FFN
        dy = dx.reshape(-1, d)
        gb["ffn"]["b2"] = dy.sum(0)
        gb["ffn"]["W2"] = c["gu"].T @ bf16_round(dy)
        dgu = bf16_round(dy) @ bf16_round(blk["ffn"]["W2"]).T
        du = _gelu_bwd(dgu, c["u"], c["t"])
        gb["ffn"]["b1"] = du.sum(0)
        gb["ffn"]["W1"] = c["h2"].reshape(-1, d).T @ bf16_round(du)
        dh2 = (bf16_round(du) @ bf16_round(blk["ffn"]["W1"]).T).reshape(bs, S, d)
        dln2, gb["ln2"]["gamma"], gb["ln2"]["beta"] = _ln_bwd(dh2, blk["ln2"]["gamma"], c["ln2"])
        dx1 = dx + dln2
        # attention
        dyo = dx1.reshape(-1, d)
        gb["attn"]["W_o"] = c["a"].reshape(-1, d).T @ bf16_round(dyo)
        da = (bf16_round(dyo) @ bf16_round(blk["attn"]["W_o"]).T).reshape(bs, S, H, dh).transpose(0, 2, 1, 3)
        pr, q, k, v = c["pr"], c["q"], c["k"], c["v"]
        dq, dk, dv = _attention_bwd(q, k, v, pr, np.ascontiguousarray(da), scale)
        dqkv = np.stack([t_.transpose(0, 2, 1, 3) for t_ in (dq, dk, dv)], axis=2).reshape(-1, 3 * d)
        gb["attn"]["W_qkv"] = c["h"].reshape(-1, d).T @ bf16_round(dqkv)
        dh1 = (bf16_round(dqkv) @ bf16_round(blk["attn"]["W_qkv"]).T).reshape(bs, S, d)
        dln1, gb["ln1"]["gamma"], gb["ln1"]["beta"] = _ln_bwd(dh1, blk["ln1"]["gamma"], c["ln1"])
        dx = dx1 + dln1
    np.add.at(G["embeddings"]["token_embed"], ids.reshape(-1), dx.reshape(-1, d))
    G["embeddings"]["pos_embed"][:S] = dx.sum(0)
    return loss, G


def warmup_cosine(count, peak, warmup, decay_steps, end):
    """optax.warmup_cosine_decay_schedule(0, peak, warmup, decay_steps, end)(count)."""
    if warmup > 0 and count < warmup:
        return peak * count / warmup
    span = max(decay_steps - warmup, 1)
    frac = min(max(count - warmup, 0), span) / span
    return end + (peak - end) * 0.5 * (1.0 + math.cos(math.pi * frac))


def global_norm(grads) -> float:
    """optax.global_norm: sqrt of the sum of squares over every leaf."""
    return float(np.sqrt(sum(float(np.sum(np.square(g, dtype=np.float64))) for g in _leaves(grads))))


def clip_by_global_norm(grads, max_norm: float):
    """optax.clip_by_global_norm(max_norm) (train.py:505-506): the leaves as they
    are while the global norm is below max_norm, else (g / norm) * max_norm."""
    n = global_norm(grads)
    if n < max_norm:
        return grads
    return _map(lambda g: (g / g.dtype.type(n)) * g.dtype.type(max_norm), grads)


class AdamWNP:
    """optax.adamw: bias-corrected Adam plus decoupled decay lr*wd*p on every leaf;
    clip_norm > 0 chains optax.clip_by_global_norm in front (train.py:502-506)."""

    def __init__(self, params, schedule, wd=0.1, b1=0.9, b2=0.999, eps=1e-8, clip_norm=0.0):
        self.schedule, self.wd, self.b1, self.b2, self.eps = schedule, wd, b1, b2, eps
        self.clip_norm = clip_norm
        self.m = [np.zeros_like(p) for p in _leaves(params)]
        self.v = [np.zeros_like(p) for p in _leaves(params)]
        self.count = 0

    def step(self, params, grads):
        if self.clip_norm > 0:
            grads = clip_by_global_norm(grads, self.clip_norm)
        lr = self.schedule(self.count)
        t = self.count + 1
        bc1, bc2 = 1 - self.b1 ** t, 1 - self.b2 ** t
        for p, g, m, v in zip(_leaves(params), _leaves(grads), self.m, self.v):
            m *= self.b1
            m += (1 - self.b1) * g
            v *= self.b2
            v += (1 - self.b2) * g * g
            p -= lr * ((m / bc1) / (np.sqrt(v / bc2) + self.eps) + self.wd * p)
        self.count = t


class MultiStepsNP:
    """optax.MultiSteps(inner, every_k_schedule=k) (train.py:319-325,507-508):
    each call is a micro-step whose gradients join the running mean
    acc + (g - acc) / (i + 1); every k-th call applies the inner optimizer to
    that mean and resets it. The inner count (the schedule) advances per update."""

    def __init__(self, inner: AdamWNP, k: int):
        self.inner, self.k = inner, k
        self.acc = None
        self.mini_step = 0

    def step(self, params, grads):
        if self.mini_step == 0:
            self.acc = _map(lambda g: g.copy(), grads)
        else:
            n = self.mini_step + 1
            self.acc = _zip_map(lambda a, g: a + (g - a) / a.dtype.type(n), self.acc, grads)
        if self.mini_step + 1 == self.k:
            self.inner.step(params, self.acc)
            self.mini_step = 0
        else:
            self.mini_step += 1


def _zip_map(fn, a, b):
    if isinstance(a, dict):
        return {k: _zip_map(fn, a[k], b[k]) for k in a}
    if isinstance(a, list):
        return [_zip_map(fn, x, y) for x, y in zip(a, b)]
    return fn(a, b)


class TrainStepNP:
    """One full training step (loss + grads + optimizer) on the CPU; with
    accum > 1 one call is one micro-step of optax.MultiSteps."""

    def __init__(self, params, lr=3e-4, warmup=0, decay_steps=1000, cfg: Config = BASELINE, wd=0.1, accum=1,
                 clip_norm=0.0):
        self.params, self.cfg = params, cfg
        sched = (lambda c: lr) if warmup == 0 and decay_steps == 0 else (
            lambda c: warmup_cosine(c, lr, warmup, decay_steps, lr / 10))
        self.opt = AdamWNP(params, sched, wd=wd, clip_norm=clip_norm)
        if accum > 1:
            self.opt = MultiStepsNP(self.opt, accum)

    def __call__(self, batch):
        loss, grads = loss_and_grads(self.params, batch, self.cfg)
        self.opt.step(self.params, grads)
        return loss
