"""nlearn_amd.attention — causal FlashAttention on gfx950 (mirrors nlearn/attention.py).

Public entry points (same names and argument meaning as the reference):

* ``attention(Q, K, V)``             Q, K, V: (n_heads, seq, d_head) -> O (attention.py:188-199)
* ``_attention_iree_flash(Q, K, V)`` the flash custom_vjp (attention.py:94-131); here a
                                     torch.autograd.Function over the HIP kernels
* ``_flash_fwd_raw(Q, K, V)``        -> (O, L) (attention.py:82-91)

Boundary dtype is bf16 (the reference upcast Q/K/V/dO to fp32 before its
kernels, attention.py:96-99,115; the kernels compute in fp32 internally).
scale = 1/sqrt(d_head) as in flash_attention.metal:64. The backward's
D = rowsum(dO * O) (attention.py:116) runs as a HIP preprocess kernel.

Beyond the reference:

* ``flash_attention(q, k, v)`` takes (B, H, S, D) views with ANY batch/head/row
  strides (unit stride along D), so head-folding transposes
  (model.py:173-198) are not needed;
* ``flash_attention_qkv(qkv)`` consumes the fused projection output
  (B, S, 3, H, D) in place and returns O laid out as (B, S, H*D); its backward
  writes dQ/dK/dV straight into one (B, S, 3, H, D) gradient.

There is no fallback path: the HIP library is required.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from .kernels import wgrad
from .kernels.gemm import _check_device

_BF16 = torch.bfloat16
PLATFORM = "rocm"


def _stride4(t: torch.Tensor) -> _lib.AttnStride:
    """(B, H, S, D) view -> nl_attn_stride (element strides)."""
    if t.stride(3) != 1:
        raise ValueError("flash attention operands need a unit stride along d_head")
    return _lib.AttnStride(t.stride(0), t.stride(1), t.stride(2))


def _ok(t: torch.Tensor) -> bool:
    return (t.stride(3) == 1 and t.data_ptr() % 16 == 0
            and all(s % 8 == 0 for s in (t.stride(0), t.stride(1), t.stride(2))) and t.stride(2) >= 64)


def _prep(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != _BF16:
        t = t.to(_BF16)
    return t if _ok(t) else t.contiguous()


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _new_bshd(B, H, S, D, device):
    """(B, H, S, D) view over (B, S, H, D) storage (the token-major layout the
    output projection reads)."""
    return torch.empty((B, S, H, D), dtype=_BF16, device=device).permute(0, 2, 1, 3)


def flash_fwd_raw4(q, k, v, causal=True, scale=None, out=None):
    """O (B,H,S,D) bf16 and L (B,H,S) fp32 natural-log logsumexp."""
    _check_device(q, k, v)
    q, k, v = _prep(q), _prep(k), _prep(v)
    B, H, S, D = q.shape
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError("flash attention: Q, K, V shapes differ")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    O = _new_bshd(B, H, S, D, q.device) if out is None else out
    L = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    _lib.call("nl_flash_attention_fwd", _stream(q), B, H, S, D, scale, int(bool(causal)),
              q.data_ptr(), _stride4(q), k.data_ptr(), _stride4(k), v.data_ptr(), _stride4(v),
              O.data_ptr(), _stride4(O), L.data_ptr())
    return O, L


def flash_bwd_raw4(q, k, v, O, dO, L, causal=True, scale=None, dq=None, dk=None, dv=None):
    """dQ, dK, dV (B,H,S,D) bf16 from the saved forward state."""
    q, k, v, O, dO = (_prep(t) for t in (q, k, v, O, dO))
    B, H, S, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    dq = _new_bshd(B, H, S, D, q.device) if dq is None else dq
    dk = _new_bshd(B, H, S, D, q.device) if dk is None else dk
    dv = _new_bshd(B, H, S, D, q.device) if dv is None else dv
    ws = torch.empty(max(_lib.ws_bytes(B, H, S), 16) // 4, dtype=torch.float32, device=q.device)
    L = L.contiguous()
    if not wgrad.active():
        _lib.call("nl_flash_attention_bwd", _stream(q), B, H, S, D, scale, int(bool(causal)),
                  q.data_ptr(), _stride4(q), k.data_ptr(), _stride4(k), v.data_ptr(), _stride4(v),
                  O.data_ptr(), _stride4(O), dO.data_ptr(), _stride4(dO), L.data_ptr(),
                  dq.data_ptr(), _stride4(dq), dk.data_ptr(), _stride4(dk), dv.data_ptr(), _stride4(dv),
                  ws.data_ptr())
        return dq, dk, dv
    # inside a training step: the same three kernels (attention.py:116, then the
    # dK/dV and dQ kernels), with dQ on a second stream beside dK/dV
    c = int(bool(causal))
    _lib.call("nl_flash_attention_bwd_preprocess", _stream(q), B, H, S, D, O.data_ptr(), _stride4(O),
              dO.data_ptr(), _stride4(dO), ws.data_ptr())
    common = (scale, c, q.data_ptr(), _stride4(q), k.data_ptr(), _stride4(k), v.data_ptr(), _stride4(v),
              dO.data_ptr(), _stride4(dO), L.data_ptr(), ws.data_ptr())
    wgrad.split(
        lambda: _lib.call("nl_flash_attention_bwd_dkdv", _stream(q), B, H, S, D, *common,
                          dk.data_ptr(), _stride4(dk), dv.data_ptr(), _stride4(dv)),
        lambda: _lib.call("nl_flash_attention_bwd_dq", _stream(q), B, H, S, D, *common, dq.data_ptr(),
                          _stride4(dq)),
        q, k, v, dO, L, ws, dq)
    return dq, dk, dv


class _Flash4(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, causal, scale):
        O, L = flash_fwd_raw4(q, k, v, causal, scale)
        ctx.save_for_backward(q, k, v, O, L)
        ctx.causal, ctx.scale = causal, scale
        return O

    @staticmethod
    def backward(ctx, dO):
        q, k, v, O, L = ctx.saved_tensors
        dq, dk, dv = flash_bwd_raw4(q, k, v, O, dO, L, ctx.causal, ctx.scale)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None


def flash_attention(q, k, v, causal: bool = True, scale: float | None = None):
    """Differentiable attention over (B, H, S, 64) views (any strides, unit along d)."""
    return _Flash4.apply(q, k, v, causal, scale)


class _FlashQKV(torch.autograd.Function):
    """Attention straight from the fused projection output qkv (B, S, 3, H, D)."""

    @staticmethod
    def forward(ctx, qkv, causal, scale):
        B, S, three, H, D = qkv.shape
        assert three == 3
        q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))
        O, L = flash_fwd_raw4(q, k, v, causal, scale)
        ctx.save_for_backward(qkv, O, L)
        ctx.causal, ctx.scale = causal, scale
        return O.permute(0, 2, 1, 3).reshape(B, S, H * D)  # storage is already (B, S, H, D)

    @staticmethod
    def backward(ctx, dO):
        qkv, O, L = ctx.saved_tensors
        B, S, _, H, D = qkv.shape
        q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))
        dO4 = dO.reshape(B, S, H, D).permute(0, 2, 1, 3)
        dqkv = torch.empty_like(qkv)
        dq, dk, dv = (dqkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))
        flash_bwd_raw4(q, k, v, O, dO4, L, ctx.causal, ctx.scale, dq=dq, dk=dk, dv=dv)
        return dqkv, None, None


def flash_attention_qkv(qkv: torch.Tensor, causal: bool = True, scale: float | None = None) -> torch.Tensor:
    """qkv: (B, S, 3, H, D) bf16 -> O: (B, S, H*D) bf16."""
    if qkv.dtype != _BF16 or not qkv.is_contiguous():
        qkv = qkv.to(_BF16).contiguous()
    return _FlashQKV.apply(qkv, causal, scale)


# ---------------------------------------------------------------------------
# reference-shaped API: (n, s, d)
# ---------------------------------------------------------------------------


def _flash_fwd_raw(Q, K, V):
    """(n,s,d) -> O (n,s,d) bf16, L (n,s) fp32 logsumexp (attention.py:82-91)."""
    O, L = flash_fwd_raw4(Q[:, None], K[:, None], V[:, None])
    return O[:, 0], L[:, 0]


def _attention_iree_flash(Q, K, V):
    """Causal flash attention, (n, s, d) -> (n, s, d) in Q's dtype (attention.py:94-131)."""
    in_dtype = Q.dtype
    O = flash_attention(Q[:, None], K[:, None], V[:, None])[:, 0]
    return O if in_dtype == _BF16 else O.to(in_dtype)


def attention(Q, K, V):
    """Q, K, V: (n_heads, seq_len, d_head) -> (n_heads, seq_len, d_head), causal."""
    return _attention_iree_flash(Q, K, V)


def print_attention_config():
    print(f"  Platform:  {PLATFORM}")
    print("  Attention: HIP FlashAttention (gfx950 MFMA kernels)")
