"""nlearn_amd.kernels.fused — the model's non-GEMM layers on the HIP kernels.

* ``layer_norm(x, gamma, beta)`` and ``add_layer_norm(x, r, gamma, beta)``:
  LayerNorm with fp32 statistics (nlearn/model.py:228-241), the second one
  with the residual add of the block folded in (model.py:315-324): it returns
  both LN(x + r) and the new residual stream x + r, reading x and r once.
* ``ffn(x, W1, b1, W2, b2)``: the FFN (model.py:266-277, with the benchmark's
  tanh-GELU and biases) as two GEMMs whose epilogues add the biases and apply
  the GELU; the backward's dX GEMM applies the GELU derivative in its
  epilogue, so no elementwise kernel runs between the GEMMs.
* ``embedding(ids, tok, pos)``: token + learned-position lookup (model.py:75-85);
  ``embedding_layer_norm`` is the lookup together with the first LayerNorm.

Every op is an autograd Function whose forward and backward are C-ABI calls;
there is no framework fallback.
"""
from __future__ import annotations

import contextlib

import torch

from .. import _lib
from . import wgrad
from .gemm import (EPI_BIAS, EPI_BIAS_GELU, EPI_DGELU, _check_device, _kernel_ready, _ld, bf16_shadow, gemm_raw,
                   grad_buffer, padded_empty, weight_grad)

_BF16 = torch.bfloat16
_F32 = torch.float32


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _rows(x: torch.Tensor) -> torch.Tensor:
    """Dense bf16 [rows, D] view of x (copies only if x is not already one)."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype != _BF16:
        x2 = x2.to(_BF16)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


def _param(p: torch.Tensor) -> torch.Tensor:
    p = p.detach()
    if p.dtype != _F32:
        p = p.to(_F32)
    return p.contiguous()


# ---------------------------------------------------------------------------
# LayerNorm
# ---------------------------------------------------------------------------


def layer_norm_fwd_raw(x2, gamma, beta, eps, residual=None):
    """-> y, s, mean, rstd with s = bf16(x + residual) (None without a residual)."""
    _check_device(x2, gamma, beta)
    rows, D = x2.shape
    y = torch.empty_like(x2)
    s = torch.empty_like(x2) if residual is not None else None
    mean = torch.empty(rows, dtype=_F32, device=x2.device)
    rstd = torch.empty(rows, dtype=_F32, device=x2.device)
    _lib.call("nl_layernorm_fwd", _stream(x2), rows, D, x2.data_ptr(),
              residual.data_ptr() if residual is not None else None, s.data_ptr() if s is not None else None,
              gamma.data_ptr(), beta.data_ptr(), float(eps), y.data_ptr(), mean.data_ptr(), rstd.data_ptr())
    return y, s, mean, rstd


_ln_defer: dict | None = None   # set inside defer_layer_norm_param_sums()


@contextlib.contextmanager
def defer_layer_norm_param_sums():
    """Inside the block, a LayerNorm backward that writes dgamma / dbeta into
    main_grad buffers leaves them as partial rows, which the next such
    backward's kernel launch reduces (nl_layernorm_bwd_deferred); leaving the
    block reduces the last ones (nl_layernorm_param_sums). The buffers are
    complete only after the block, so it belongs around a backward pass whose
    parameter gradients an optimizer reads afterwards. The sums are the same
    bit for bit; the chain of 9 LayerNorm backwards loses 8 kernel launches.
    Module-global like kernels.wgrad (the autograd engine runs the backward
    on its own thread); one block at a time."""
    global _ln_defer
    if _ln_defer is not None:
        raise RuntimeError("defer_layer_norm_param_sums() does not nest")
    _ln_defer = {"pending": None}
    try:
        yield
    finally:
        pending, _ln_defer = _ln_defer["pending"], None
        if pending is not None:
            stream, ws, rows, D, dg, db = pending
            _lib.call("nl_layernorm_param_sums", stream, rows, D, ws.data_ptr(), dg.data_ptr(), db.data_ptr(), 0)


def layer_norm_bwd_raw(dy2, xin, mean, rstd, gamma, dres=None, dgamma=None, dbeta=None):
    """-> dx (+ dres), dgamma, dbeta (written into the given buffers if any;
    deferred inside ``defer_layer_norm_param_sums`` when both are given)."""
    rows, D = dy2.shape
    dx = torch.empty_like(dy2)
    wsb = int(_lib.load().nl_layernorm_bwd_ws_bytes(rows, D))
    ws = torch.empty(max(wsb, 16) // 4, dtype=_F32, device=dy2.device)
    dres_ptr = dres.data_ptr() if dres is not None else None
    if _ln_defer is not None and dgamma is not None and dbeta is not None:
        prev = _ln_defer["pending"]
        stream = _stream(dy2)
        if prev is not None and prev[0] != stream:
            raise RuntimeError("layer_norm backward: deferred parameter sums on two streams")
        pargs = (prev[2], prev[3], prev[1].data_ptr(), prev[4].data_ptr(), prev[5].data_ptr(), 0) if prev else \
            (0, 0, None, None, None, 0)
        _lib.call("nl_layernorm_bwd_deferred", stream, rows, D, dy2.data_ptr(), xin.data_ptr(), mean.data_ptr(),
                  rstd.data_ptr(), gamma.data_ptr(), dres_ptr, dx.data_ptr(), ws.data_ptr(), wsb, *pargs)
        # the previous partials are read by the launch just queued: stream order
        # keeps their memory from being reused before it runs
        _ln_defer["pending"] = (stream, ws, rows, D, dgamma, dbeta)
        return dx, dgamma, dbeta
    if dgamma is None:
        dgamma = torch.empty(D, dtype=_F32, device=dy2.device)
    if dbeta is None:
        dbeta = torch.empty(D, dtype=_F32, device=dy2.device)
    _lib.call("nl_layernorm_bwd", _stream(dy2), rows, D, dy2.data_ptr(), xin.data_ptr(), mean.data_ptr(),
              rstd.data_ptr(), gamma.data_ptr(), dres_ptr, dx.data_ptr(), dgamma.data_ptr(), dbeta.data_ptr(), 0,
              ws.data_ptr(), wsb)
    return dx, dgamma, dbeta


class _LayerNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gamma, beta, eps):
        x2 = _rows(x)
        g, b = _param(gamma), _param(beta)
        y, _, mean, rstd = layer_norm_fwd_raw(x2, g, b, eps)
        ctx.save_for_backward(x2, mean, rstd, g)
        ctx.shape = x.shape
        ctx.bufs = (grad_buffer(gamma), grad_buffer(beta))
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2, mean, rstd, g = ctx.saved_tensors
        dx, dg, db = layer_norm_bwd_raw(_rows(dy), x2, mean, rstd, g, None, *ctx.bufs)
        return dx.view(ctx.shape), *_unless_buffered(ctx.bufs, (dg, db)), None


class _AddLayerNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, r, gamma, beta, eps):
        ctx.set_materialize_grads(False)
        x2, r2 = _rows(x), _rows(r)
        if x2.shape != r2.shape:
            raise ValueError("add_layer_norm: x and r differ in shape")
        g, b = _param(gamma), _param(beta)
        y, s, mean, rstd = layer_norm_fwd_raw(x2, g, b, eps, residual=r2)
        ctx.save_for_backward(s, mean, rstd, g)
        ctx.shape = x.shape
        ctx.bufs = (grad_buffer(gamma), grad_buffer(beta))
        return y.view(x.shape), s.view(x.shape)

    @staticmethod
    def backward(ctx, dy, ds):
        s, mean, rstd, g = ctx.saved_tensors
        if dy is None:
            dx = _rows(ds)
            return dx.view(ctx.shape), dx.view(ctx.shape), None, None, None
        dx, dg, db = layer_norm_bwd_raw(_rows(dy), s, mean, rstd, g, _rows(ds) if ds is not None else None,
                                        *ctx.bufs)
        dx = dx.view(ctx.shape)
        return dx, dx, *_unless_buffered(ctx.bufs, (dg, db)), None


def _wgrad(X, dY, buf):
    """X^T . dY into the gradient buffer (forked when overlapping), or a fresh fp32 tensor."""
    if buf is not None:
        return weight_grad(X, dY, buf)
    return gemm_raw(X, dY, "T", "N", out_dtype=_F32)


def _unless_buffered(bufs, grads):
    """Gradients to hand back to autograd: None where a main_grad buffer took them."""
    return tuple(None if b is not None else g for b, g in zip(bufs, grads))


def layer_norm(x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """bf16 LayerNorm over the last dimension, fp32 statistics and parameters."""
    return _LayerNorm.apply(x, gamma, beta, eps)


def add_layer_norm(x: torch.Tensor, r: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor,
                   eps: float = 1e-5):
    """(LN(s), s) with s = bf16(x + r): the residual add and the next LayerNorm in one pass."""
    return _AddLayerNorm.apply(x, r, gamma, beta, eps)


# ---------------------------------------------------------------------------
# bias gradients
# ---------------------------------------------------------------------------


def colsum(x2: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 column sums of a bf16 [rows, cols] matrix (fixed summation order).

    With a preallocated ``out`` (a bias gradient buffer) the kernels are forked
    onto the weight-gradient stream when one is active (kernels.wgrad)."""
    rows, cols = x2.shape
    x2 = _kernel_ready(x2)
    fresh = out is None
    if fresh:
        out = torch.empty(cols, dtype=_F32, device=x2.device)
    wsb = int(_lib.load().nl_colsum_ws_bytes(rows, cols))
    ws = torch.empty(max(wsb, 16) // 4, dtype=_F32, device=x2.device)

    def run():
        _lib.call("nl_colsum_bf16", _stream(x2), rows, cols, x2.data_ptr(), _ld(x2), out.data_ptr(), 0,
                  ws.data_ptr(), wsb)
        return out

    return run() if fresh else wgrad.fork(run, x2, out, ws)


# ---------------------------------------------------------------------------
# FFN
# ---------------------------------------------------------------------------


class _FFN(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, W1, b1, W2, b2):
        x2 = _rows(x)
        W1b, W2b = bf16_shadow(W1), bf16_shadow(W2)
        b1f, b2f = _param(b1), _param(b2)
        M, F_ = x2.shape[0], W1b.shape[1]
        u = padded_empty(M, F_, _BF16, x2.device)         # pre-activation, kept for the backward
        h = padded_empty(M, F_, _BF16, x2.device)         # gelu(u)
        gemm_raw(x2, W1b, out=h, epi=EPI_BIAS_GELU, bias=b1f, aux=u)
        y = padded_empty(M, W2b.shape[1], _BF16, x2.device)
        gemm_raw(h, W2b, out=y, epi=EPI_BIAS, bias=b2f)
        ctx.save_for_backward(x2, u, h)
        ctx.wb = (W1b, W2b)
        ctx.bufs = tuple(grad_buffer(t) for t in (W1, b1, W2, b2))
        ctx.shape = x.shape
        return y.view(*x.shape[:-1], W2b.shape[1])

    @staticmethod
    def backward(ctx, dy):
        x2, u, h = ctx.saved_tensors
        W1b, W2b = ctx.wb
        gW1, gb1, gW2, gb2 = ctx.bufs
        dy2 = _rows(dy)
        db2 = colsum(dy2, out=gb2)
        dW2 = _wgrad(h, dy2, gW2)                                                  # h^T . dy
        du = padded_empty(u.shape[0], u.shape[1], _BF16, dy2.device)
        gemm_raw(dy2, W2b, "N", "T", out=du, epi=EPI_DGELU, aux=u)               # (dy . W2^T) * gelu'(u)
        db1 = colsum(du, out=gb1)
        dW1 = _wgrad(x2, du, gW1)                                                  # x^T . du
        dx = gemm_raw(du, W1b, "N", "T", out_dtype=_BF16)                          # du . W1^T
        return dx.view(ctx.shape), *_unless_buffered(ctx.bufs, (dW1, db1, dW2, db2))


def ffn(x: torch.Tensor, W1: torch.Tensor, b1: torch.Tensor, W2: torch.Tensor, b2: torch.Tensor) -> torch.Tensor:
    """gelu_tanh(x @ W1 + b1) @ W2 + b2 in bf16 with fp32 accumulation."""
    return _FFN.apply(x, W1, b1, W2, b2)


# ---------------------------------------------------------------------------
# embedding
# ---------------------------------------------------------------------------


def _embedding_fwd(ids, tok, pos):
    """-> (bf16 (B, S, D) lookup, int32 ids, dims for the backward)."""
    B, S = ids.shape
    V, D = tok.shape
    if S > pos.shape[0]:
        raise ValueError(f"embedding: sequence {S} exceeds the position table ({pos.shape[0]})")
    ids32 = ids.to(torch.int32).contiguous()
    t, p = _param(tok), _param(pos)
    _check_device(ids32, t, p)
    out = torch.empty((B, S, D), dtype=_BF16, device=ids.device)
    _lib.call("nl_embedding_fwd", _stream(out), B, S, D, V, ids32.data_ptr(), t.data_ptr(), p.data_ptr(),
              out.data_ptr())
    return out, ids32, (B, S, D, V, tuple(pos.shape))


class _Embedding(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ids, tok, pos):
        out, ids32, ctx.dims = _embedding_fwd(ids, tok, pos)
        ctx.save_for_backward(ids32)
        ctx.bufs = (grad_buffer(tok), grad_buffer(pos))
        return out

    @staticmethod
    def backward(ctx, dx):
        (ids32,) = ctx.saved_tensors
        return None, *_embedding_bwd(ids32, dx, ctx.dims, ctx.bufs)


def _embedding_bwd(ids32, dx, dims, bufs):
    """(dtok, dpos) of the lookup, None where a main_grad buffer took them."""
    B, S, D, V, pshape = dims
    dx = dx.to(_BF16).contiguous()
    gt, gp = bufs
    # the kernel writes every row of dtok (zero where no token has the id); of
    # dpos it writes rows [0, S), so only a longer table needs a fill (zero_()
    # is a fill kernel: no memset node when the step is captured)
    dtok = gt if gt is not None else torch.empty((V, D), dtype=_F32, device=dx.device)
    if gp is None:
        dpos = torch.zeros(pshape, dtype=_F32, device=dx.device)
    else:
        dpos = gp.zero_() if pshape[0] > S else gp
    wsb = int(_lib.load().nl_embedding_bwd_ws_bytes(B, S, D, V))
    ws = torch.empty(max(wsb, 16) // 4, dtype=torch.int32, device=dx.device)
    _lib.call("nl_embedding_bwd", _stream(dx), B, S, D, V, ids32.data_ptr(), dx.data_ptr(), dtok.data_ptr(),
              dpos.data_ptr(), 0, ws.data_ptr(), wsb)
    return _unless_buffered(bufs, (dtok, dpos))


def embedding(ids: torch.Tensor, tok: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
    """bf16 (B, S, D) = tok[ids] + pos[:S] for int ids (B, S)."""
    return _Embedding.apply(ids, tok, pos)


class _EmbeddingLayerNorm(torch.autograd.Function):
    """The lookup and the first block's LayerNorm as one node: the residual
    stream x and LN(x) both leave it, so in the backward the LayerNorm kernel
    adds x's other gradient (dres) while forming its own, and the lookup's
    backward reads the sum (no separate add of the two gradients)."""

    @staticmethod
    def forward(ctx, ids, tok, pos, gamma, beta, eps):
        ctx.set_materialize_grads(False)
        x, ids32, ctx.dims = _embedding_fwd(ids, tok, pos)
        x2 = x.view(-1, x.shape[-1])
        g, b = _param(gamma), _param(beta)
        y, _, mean, rstd = layer_norm_fwd_raw(x2, g, b, eps)
        ctx.save_for_backward(ids32, x2, mean, rstd, g)
        ctx.bufs = (grad_buffer(tok), grad_buffer(pos))
        ctx.ln_bufs = (grad_buffer(gamma), grad_buffer(beta))
        return y.view(x.shape), x2.view(x.shape)

    @staticmethod
    def backward(ctx, dy, dx):
        ids32, x2, mean, rstd, g = ctx.saved_tensors
        ln_grads = (None, None)
        if dy is not None:
            dx2, dg, db = layer_norm_bwd_raw(_rows(dy), x2, mean, rstd, g, _rows(dx) if dx is not None else None,
                                             *ctx.ln_bufs)
            dx = dx2
            ln_grads = _unless_buffered(ctx.ln_bufs, (dg, db))
        if dx is None:
            return None, None, None, *ln_grads, None
        return None, *_embedding_bwd(ids32, dx, ctx.dims, ctx.bufs), *ln_grads, None


def embedding_layer_norm(ids: torch.Tensor, tok: torch.Tensor, pos: torch.Tensor, gamma: torch.Tensor,
                         beta: torch.Tensor, eps: float = 1e-5):
    """(LN(x), x) with x = embedding(ids, tok, pos): the lookup and the first
    LayerNorm, whose backward also takes in x's residual-stream gradient."""
    return _EmbeddingLayerNorm.apply(ids, tok, pos, gamma, beta, eps)
