"""nlearn_amd.model — the BASELINE GPT-style decoder, built on the HIP kernels.

Caller of the hot path, mirroring nlearn/model.py's structure and names
(``init_model``, ``model_forward_features``, ``model_forward``,
``output_projection``) with the architecture BASELINE.json specifies (the
reference's current model.py is a larger RMSNorm/RoPE/SwiGLU variant; its
docstrings at model.py:249-252,303 describe this older layout):

    d_model 512, 8 heads of 64, 4 layers, FFN 2048 with tanh-GELU (+biases),
    pre-LayerNorm (gamma=1, beta=0), learned positions, untied LM head,
    vocab 50257  ->  64.3 M parameters.

Parameters are fp32 masters (model.py:372-375 keeps f32 params and casts to
the bf16 compute dtype); every GEMM reads a bf16 shadow of its weight. The
three projections W_q, W_k, W_v are stored as one [d, 3d] matrix (column
blocks q | k | v) so QKV is one GEMM whose output feeds the flash kernel in
place: the head-folding transposes of model.py:173-198 disappear.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from .attention import flash_attention_qkv
from .kernels import fused
from .kernels.gemm import linear

COMPUTE_DTYPE = torch.bfloat16


@dataclass(frozen=True)
class ModelConfig:
    vocab_size: int = 50257
    d_model: int = 512
    n_heads: int = 8
    n_layers: int = 4
    d_ff: int = 2048
    max_seq_len: int = 512
    ln_eps: float = 1e-5

    @property
    def d_head(self) -> int:
        return self.d_model // self.n_heads


BASELINE = ModelConfig()


def param_shapes(cfg: ModelConfig = BASELINE) -> dict:
    """Nested dict of parameter shapes (the checkpoint layout)."""
    d, f = cfg.d_model, cfg.d_ff
    block = {
        "ln1": {"gamma": (d,), "beta": (d,)},
        "attn": {"W_qkv": (d, 3 * d), "W_o": (d, d)},
        "ln2": {"gamma": (d,), "beta": (d,)},
        "ffn": {"W1": (d, f), "b1": (f,), "W2": (f, d), "b2": (d,)},
    }
    return {
        "embeddings": {"token_embed": (cfg.vocab_size, d), "pos_embed": (cfg.max_seq_len, d)},
        "blocks": [block for _ in range(cfg.n_layers)],
        "ln_final": {"gamma": (d,), "beta": (d,)},
        "lm_head": (d, cfg.vocab_size),
    }


def tree_map(fn, tree):
    if isinstance(tree, dict):
        return {k: tree_map(fn, v) for k, v in tree.items()}
    if isinstance(tree, list):
        return [tree_map(fn, v) for v in tree]
    return fn(tree)


def tree_leaves(tree) -> list:
    if isinstance(tree, dict):
        return [x for k in tree for x in tree_leaves(tree[k])]
    if isinstance(tree, list):
        return [x for v in tree for x in tree_leaves(v)]
    return [tree]


def tree_paths(tree, prefix=()) -> list:
    if isinstance(tree, dict):
        return [p for k in tree for p in tree_paths(tree[k], prefix + (k,))]
    if isinstance(tree, list):
        return [p for i, v in enumerate(tree) for p in tree_paths(v, prefix + (i,))]
    return [prefix]


def init_params_numpy(seed: int = 0, cfg: ModelConfig = BASELINE) -> dict:
    """fp32 NumPy parameters: weights N(0, 0.02), LayerNorm gamma 1 / beta 0,
    biases 0 (model.py:63-70,112-132,221-226 initialise with the same law)."""
    rng = np.random.default_rng(seed)

    def make(path_shape):
        path, shape = path_shape
        name = path[-1]
        if name == "gamma":
            return np.ones(shape, np.float32)
        if name in ("beta", "b1", "b2"):
            return np.zeros(shape, np.float32)
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).astype(np.float32)

    shapes = param_shapes(cfg)
    paths = tree_paths(shapes)
    leaves = [make((p, s)) for p, s in zip(paths, tree_leaves(shapes))]
    it = iter(leaves)
    return tree_map(lambda _: next(it), shapes)


def device_param(a: np.ndarray, device="cuda") -> torch.Tensor:
    """A leaf parameter on the device. A matrix whose row is not a whole number
    of 16-byte chunks (the LM head: 50257 columns) is stored with its row
    stride rounded up to 8 elements, so the GEMMs, the gradient buffer and the
    optimizer all address it with aligned rows; the padding stays zero."""
    t = torch.from_numpy(np.ascontiguousarray(a))
    if t.dim() == 2 and t.shape[1] % 8:
        rows, cols = t.shape
        base = torch.zeros((rows, (cols + 7) // 8 * 8), dtype=t.dtype, device=device)
        base[:, :cols] = t.to(device)
        return base[:, :cols].requires_grad_(True)
    return t.to(device).requires_grad_(True)


def init_model(seed: int = 0, cfg: ModelConfig = BASELINE, device="cuda") -> dict:
    """fp32 device parameters, requires_grad, seeded through NumPy so a CPU
    restatement can start from the identical weights."""
    return tree_map(lambda a: device_param(a, device), init_params_numpy(seed, cfg))


def count_params(params) -> int:
    return sum(int(np.prod(p.shape)) for p in tree_leaves(params))


# ---------------------------------------------------------------------------
# forward
# ---------------------------------------------------------------------------


def embed(params, token_ids: torch.Tensor) -> torch.Tensor:
    """token + learned position embeddings -> bf16 (bs, seq, d) (one HIP kernel)."""
    e = params["embeddings"]
    return fused.embedding(token_ids, e["token_embed"], e["pos_embed"])


def layer_norm(p, x: torch.Tensor, eps: float = BASELINE.ln_eps) -> torch.Tensor:
    """Pre-LN LayerNorm with learned gamma / beta (bf16 in and out, fp32 statistics)."""
    return fused.layer_norm(x, p["gamma"], p["beta"], eps)


def attention_forward(p, x: torch.Tensor, cfg: ModelConfig) -> torch.Tensor:
    bs, s, d = x.shape
    qkv = linear(x, p["W_qkv"]).view(bs, s, 3, cfg.n_heads, cfg.d_head)
    out = flash_attention_qkv(qkv)                       # (bs, s, d), token-major
    return linear(out, p["W_o"])


def ffn_forward(p, x: torch.Tensor) -> torch.Tensor:
    """gelu_tanh(x W1 + b1) W2 + b2; bias and GELU live in the GEMM epilogues."""
    return fused.ffn(x, p["W1"], p["b1"], p["W2"], p["b2"])


def block_forward(p, x: torch.Tensor, cfg: ModelConfig) -> torch.Tensor:
    """One pre-LN block, x -> x + attn(LN1 x) -> (.) + ffn(LN2 .) (model.py:315-324)."""
    x, r = _block(p, x, None, cfg)
    return x + r


def _block(p, x: torch.Tensor, r, cfg: ModelConfig, h=None):
    """Block with its residual adds deferred: the stream arrives as x + r (r may
    be None) and leaves as (x', r'); each add is folded into the next LayerNorm.
    ``h`` is LN1(x) when the caller already formed it."""
    if h is None and r is None:
        h = layer_norm(p["ln1"], x, cfg.ln_eps)
    elif h is None:
        h, x = fused.add_layer_norm(x, r, p["ln1"]["gamma"], p["ln1"]["beta"], cfg.ln_eps)
    a = attention_forward(p["attn"], h, cfg)
    h2, x = fused.add_layer_norm(x, a, p["ln2"]["gamma"], p["ln2"]["beta"], cfg.ln_eps)
    return x, ffn_forward(p["ffn"], h2)


def model_forward_features(params, token_ids: torch.Tensor, cfg: ModelConfig = BASELINE) -> torch.Tensor:
    """Hidden states after the final LayerNorm, bf16 (bs, seq, d). The lookup
    and the first block's LN1 are one node (fused.embedding_layer_norm)."""
    blocks = params["blocks"]
    r = None
    if blocks:
        e, ln1 = params["embeddings"], blocks[0]["ln1"]
        h, x = fused.embedding_layer_norm(token_ids, e["token_embed"], e["pos_embed"], ln1["gamma"], ln1["beta"],
                                          cfg.ln_eps)
        x, r = _block(blocks[0], x, None, cfg, h=h)
    else:
        x = embed(params, token_ids)
    for bp in blocks[1:]:
        x, r = _block(bp, x, r, cfg)
    lf = params["ln_final"]
    if r is None:
        return layer_norm(lf, x, cfg.ln_eps)
    return fused.add_layer_norm(x, r, lf["gamma"], lf["beta"], cfg.ln_eps)[0]


def output_projection(params) -> torch.Tensor:
    """The untied (d_model, vocab) LM-head matrix."""
    return params["lm_head"]


def model_forward(params, token_ids: torch.Tensor, cfg: ModelConfig = BASELINE) -> torch.Tensor:
    """token ids (bs, seq) -> bf16 logits (bs, seq, vocab) (rows 16-byte aligned)."""
    x = model_forward_features(params, token_ids, cfg)
    return linear(x, output_projection(params))


def flops_per_step(cfg: ModelConfig, bs: int, seq: int) -> dict:
    """Algorithmic matmul FLOPs of one training step (forward + backward, no
    recomputation): every GEMM counted 3x (forward, dX, dW), causal attention
    2*n*s^2*d forward and 2.5x that backward."""
    M = bs * seq
    d, f, V = cfg.d_model, cfg.d_ff, cfg.vocab_size
    per_layer = 2 * M * (d * 3 * d + d * d + d * f + f * d)
    gemm = 3 * (cfg.n_layers * per_layer + 2 * M * d * V)
    n = bs * cfg.n_heads
    attn_fwd = 2 * n * seq * seq * cfg.d_head
    attn = cfg.n_layers * attn_fwd * 3.5
    return {"gemm": float(gemm), "attention": float(attn), "total": float(gemm + attn),
            "six_n_t": 6.0 * count_params_cfg(cfg) * M}


def count_params_cfg(cfg: ModelConfig) -> int:
    return sum(int(np.prod(s)) for s in tree_leaves(param_shapes(cfg)))


__all__ = [
    "ModelConfig", "BASELINE", "init_model", "init_params_numpy", "model_forward", "model_forward_features",
    "output_projection", "embed", "layer_norm", "block_forward", "tree_map", "tree_leaves", "count_params",
    "flops_per_step",
]
