"""nlearn_amd.kernels.cross_entropy — fused softmax cross-entropy on gfx950.

Mirrors nlearn/kernels/cross_entropy.py:

* ``cross_entropy(logits, targets)``: mean softmax CE over the flattened rows,
  differentiable in ``logits`` (cross_entropy.py:71-81). The forward makes ONE
  pass over the bf16 logits and produces the per-row loss, the logsumexp and
  dlogits = (softmax - onehot)/M together (the reference ran ce_fwd, then
  ce_bwd as a second pass in the backward, cross_entropy.py:55-65). With
  ``inplace=True`` dlogits overwrite the logits, so the (M, V) gradient costs
  no extra memory.
* The backward multiplies by the incoming cotangent g with a kernel that reads
  g on the device and skips the pass when g == 1 (the training loss), so no
  host synchronisation happens.
* ``_ce_fwd_raw`` / ``_ce_bwd_raw`` keep the reference's two-target form
  (cross_entropy.py:28-46) for callers that want the separate passes.
* ``linear_cross_entropy(X, W, targets)``: the LM head and the CE fused, with
  no (M, V) logits in memory between forward and backward
  (cross_entropy.py:84-170). The forward GEMM reduces its tiles of logits to
  per-row softmax statistics in the epilogue, so the logits are never stored;
  the backward recomputes them in a GEMM whose epilogue writes dlogits, for
  the whole vocabulary at once or in ``NLEARN_LCE_CHUNK``-column slices.
"""
from __future__ import annotations

import os

import torch

from .. import _lib
from . import wgrad
from .gemm import (_check_device, _kernel_ready, bf16_shadow, gemm_raw, grad_buffer, linear_backward, padded_empty,
                   weight_grad)

_BF16 = torch.bfloat16


def _as_rows(logits: torch.Tensor) -> torch.Tensor:
    V = logits.shape[-1]
    x = logits.reshape(-1, V)
    if x.stride(-1) != 1:
        raise ValueError("cross_entropy: logits need a unit stride along the vocabulary")
    if x.shape[0] > 1 and x.stride(0) < V:  # rows sharing memory (a broadcast view)
        x = x.contiguous()
    return x


def _ld(x: torch.Tensor) -> int:
    return x.stride(0) if x.shape[0] > 1 else x.shape[1]


def _targets(targets: torch.Tensor) -> torch.Tensor:
    t = targets.reshape(-1)
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ce_fwd_raw(logits: torch.Tensor, targets: torch.Tensor):
    """logits[M,V] bf16, targets[M] -> (loss[M] f32, lse[M] f32). ("ce_fwd")"""
    x = _as_rows(logits.to(_BF16))
    t = _targets(targets)
    _check_device(x, t)
    M, V = x.shape
    loss = torch.empty(M, dtype=torch.float32, device=x.device)
    lse = torch.empty(M, dtype=torch.float32, device=x.device)
    _lib.call("nl_ce_fwd", _stream(x), M, V, x.data_ptr(), _ld(x), t.data_ptr(), loss.data_ptr(), lse.data_ptr())
    return loss, lse


def _ce_bwd_raw(logits: torch.Tensor, targets: torch.Tensor, lse: torch.Tensor, scale: float | None = None):
    """dlogits[M,V] = (softmax - onehot) * scale, scale defaulting to 1/M. ("ce_bwd")"""
    x = _as_rows(logits.to(_BF16))
    t = _targets(targets)
    M, V = x.shape
    scale = (1.0 / M) if scale is None else scale
    d = torch.empty((M, V), dtype=_BF16, device=x.device)
    _lib.call("nl_ce_bwd", _stream(x), M, V, x.data_ptr(), _ld(x), t.data_ptr(), lse.contiguous().data_ptr(),
              float(scale), d.data_ptr(), _ld(d))
    return d


def ce_fwd_bwd_raw(logits: torch.Tensor, targets: torch.Tensor, inplace: bool = False, scale: float | None = None):
    """Single pass: (loss[M], lse[M], dlogits[M,V]); dlogits overwrite logits if inplace."""
    x = _as_rows(logits)
    if x.dtype != _BF16:
        raise ValueError("cross_entropy: logits must be bfloat16")
    t = _targets(targets)
    _check_device(x, t)
    M, V = x.shape
    scale = (1.0 / M) if scale is None else scale
    loss = torch.empty(M, dtype=torch.float32, device=x.device)
    lse = torch.empty(M, dtype=torch.float32, device=x.device)
    if inplace:
        d = x
    else:
        d = torch.empty((M, _ld(x)), dtype=_BF16, device=x.device)[:, :V] if M > 1 else torch.empty_like(x)
    _lib.call("nl_ce_fwd_bwd", _stream(x), M, V, x.data_ptr(), _ld(x), t.data_ptr(), loss.data_ptr(),
              lse.data_ptr(), float(scale), d.data_ptr(), _ld(d))
    return loss, lse, d


def mean(x: torch.Tensor) -> torch.Tensor:
    """Deterministic fp32 mean of a 1-D device tensor (0-d result)."""
    x = x.contiguous()
    out = torch.empty((), dtype=torch.float32, device=x.device)
    _lib.call("nl_mean_f32", _stream(x), x.data_ptr(), x.numel(), out.data_ptr())
    return out


def scale_by_device_scalar_(d: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """d *= g in place (bf16 rows), skipped on the device when g == 1."""
    g = g.reshape(()).to(torch.float32)
    rows = d.shape[0]
    _lib.call("nl_scale_bf16_by_device_scalar", _stream(d), d.data_ptr(), rows, d.shape[1], _ld(d), g.data_ptr())
    return d


class _CE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits2d, targets, inplace):
        loss_rows, lse, d = ce_fwd_bwd_raw(logits2d, targets, inplace=inplace)
        ctx.d = d
        ctx.mark_non_differentiable(lse)
        return mean(loss_rows)

    @staticmethod
    def backward(ctx, g):
        d = ctx.d
        ctx.d = None
        return scale_by_device_scalar_(d, g), None, None


def cross_entropy(logits: torch.Tensor, targets: torch.Tensor, inplace: bool = False) -> torch.Tensor:
    """Mean softmax cross-entropy of bf16 logits[..., V] against int targets[...].

    ``inplace=True`` lets the single pass write dlogits over ``logits`` (use it
    when nothing else reads the logits afterwards, as in the training step).
    """
    x = _as_rows(logits)
    out = _CE.apply(x, targets, inplace)
    return out


# ---------------------------------------------------------------------------
# LM head + cross-entropy with the CE pipelined behind the logits GEMM
# ---------------------------------------------------------------------------


# With two chunks the first takes this share of the rows (whole 256-row tiles):
# its CE then overlaps the shorter second GEMM chunk, and the CE left alone at
# the end is shorter. Measured on MI355X at bs32 x seq512 (graph replays, two
# rounds on one box): equal halves 5.887-5.894 ms per step, 55% 5.868-5.877,
# 60% 5.852-5.854, 65% 5.863; three equal chunks 5.922-5.930.
FIRST_CHUNK_SHARE = 0.6


def chunk_bounds(M: int, n: int) -> list:
    """Row boundaries of ``n`` LM-head chunks over M rows (first 0, last M)."""
    n = max(1, min(int(n), M)) if M > 0 else 1
    if n == 2 and M >= 512:
        cut = int(M * FIRST_CHUNK_SHARE) // 256 * 256
        if 0 < cut < M:
            return [0, cut, M]
    return [M * i // n for i in range(n + 1)]


class _LMHeadCE(torch.autograd.Function):
    """logits = X . W, then the single CE pass (loss, lse and dlogits written
    over the logits), in row chunks. With more than one chunk, each chunk's CE
    runs on a second stream while the GEMM computes the next chunk, so the
    HBM-bound CE overlaps the MFMA-bound GEMM. Rows are independent in both
    kernels, and the CE scale is 1/M of all rows, so every value equals the
    unchunked linear + cross_entropy bit for bit. The backward is linear's,
    from dlogits scaled by the cotangent."""

    @staticmethod
    def forward(ctx, x2, W, targets, chunks, overlap):
        Wb = bf16_shadow(W)
        M, V = x2.shape[0], Wb.shape[1]
        t = _targets(targets)
        if t.numel() != M:
            raise ValueError(f"lm_head_cross_entropy: {t.numel()} targets for {M} rows")
        _check_device(x2, t)
        logits = padded_empty(M, V, _BF16, x2.device)
        ld = _ld(logits)
        loss_rows = torch.empty(M, dtype=torch.float32, device=x2.device)
        lse = torch.empty(M, dtype=torch.float32, device=x2.device)
        main = torch.cuda.current_stream(x2.device)
        n = max(1, min(int(chunks), M))
        aux = wgrad._side_stream(x2.device, 1) if n > 1 and overlap else None
        bounds = chunk_bounds(M, n)
        for r0, r1 in zip(bounds[:-1], bounds[1:]):
            if r1 == r0:
                continue
            gemm_raw(x2[r0:r1], Wb, out=logits[r0:r1])
            ce = (lambda st, r0=r0, r1=r1: _lib.call(
                "nl_ce_fwd_bwd", st, r1 - r0, V, logits[r0].data_ptr(), ld, t[r0].data_ptr(),
                loss_rows[r0].data_ptr(), lse[r0].data_ptr(), 1.0 / M, logits[r0].data_ptr(), ld))
            if aux is None:
                ce(main.cuda_stream)
                continue
            # everything these CE launches touch was allocated above, on the
            # current stream, and stays referenced until the join below
            aux.wait_stream(main)
            with torch.cuda.stream(aux):
                ce(aux.cuda_stream)
        if aux is not None:
            main.wait_stream(aux)
        ctx.save_for_backward(x2, W)
        ctx.wb = Wb
        ctx.d = logits
        return mean(loss_rows)

    @staticmethod
    def backward(ctx, g):
        x2, W = ctx.saved_tensors
        d = ctx.d
        ctx.d = None
        scale_by_device_scalar_(d, g)
        dx, dW = linear_backward(x2, W, ctx.wb, d, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return dx, dW, None, None, None


def lm_head_cross_entropy(X: torch.Tensor, W: torch.Tensor, targets: torch.Tensor, chunks: int = 1,
                          overlap: bool = True) -> torch.Tensor:
    """Mean CE of logits = X . W (X [..., d] bf16, W [d, V]) against ``targets``,
    equal to ``cross_entropy(linear(X, W), targets, inplace=True)`` bit for
    bit; with ``chunks`` > 1 row chunks, the CE of one chunk overlaps the GEMM
    of the next (see _LMHeadCE) unless ``overlap`` is False (every kernel then
    runs on the current stream, in the same order)."""
    if X.dim() < 2 or W.dim() != 2:
        raise ValueError("lm_head_cross_entropy: X needs >= 2 dims and W exactly 2")
    x2 = X.reshape(-1, X.shape[-1])
    return _LMHeadCE.apply(x2, W, targets.reshape(-1), int(chunks), bool(overlap))


# ---------------------------------------------------------------------------
# linear_cross_entropy — cross_entropy.py:84-170
# ---------------------------------------------------------------------------

# Columns of dlogits the backward forms at a time (0: the whole vocabulary).
# The reference chunks by NLEARN_LCE_CHUNK = 4096 in both passes
# (cross_entropy.py:93); here the forward never needs chunks, and the backward
# only needs them to cap the transient dlogits buffer (M x chunk bf16).
_LCE_CHUNK = int(os.environ.get("NLEARN_LCE_CHUNK", "0"))


def _lce_chunk(V: int) -> int:
    if _LCE_CHUNK <= 0 or _LCE_CHUNK >= V:
        return V
    return max(256, _LCE_CHUNK // 256 * 256)


class _LinearCE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x2, W, targets):
        Wb = bf16_shadow(W)
        xb = _kernel_ready(x2)
        t = _targets(targets)
        _check_device(xb, Wb, t)
        M, D = xb.shape
        if Wb.shape[0] != D:
            raise ValueError(f"linear_cross_entropy: X has {D} features, W has {Wb.shape[0]} rows")
        if t.numel() != M:
            raise ValueError("linear_cross_entropy: one target per row of X")
        V = Wb.shape[1]
        loss_rows = torch.empty(M, dtype=torch.float32, device=xb.device)
        lse = torch.empty(M, dtype=torch.float32, device=xb.device)
        wsb = int(_lib.load().nl_lce_ws_bytes(M, V))
        ws = torch.empty(max(wsb, 16) // 4, dtype=torch.float32, device=xb.device)
        _lib.call("nl_lce_fwd", _stream(xb), M, D, V, xb.data_ptr(), _ld(xb), Wb.data_ptr(), _ld(Wb), t.data_ptr(),
                  loss_rows.data_ptr(), lse.data_ptr(), ws.data_ptr(), wsb)
        ctx.save_for_backward(xb, W, t, lse)
        ctx.wb = Wb
        ctx.x_dtype = x2.dtype
        return mean(loss_rows)

    @staticmethod
    def backward(ctx, g):
        xb, W, t, lse = ctx.saved_tensors
        Wb = ctx.wb
        M, D = xb.shape
        V = Wb.shape[1]
        g = g.reshape(1).to(torch.float32).contiguous()
        chunk = _lce_chunk(V)
        mg = grad_buffer(W) if ctx.needs_input_grad[1] else None
        dX = dW = None

        def dlogits(v0: int, vn: int, buf: torch.Tensor) -> torch.Tensor:
            d = buf[:, :vn]
            _lib.call("nl_lce_bwd_dlogits", _stream(xb), M, D, V, v0, vn, xb.data_ptr(), _ld(xb), Wb.data_ptr(),
                      _ld(Wb), t.data_ptr(), lse.data_ptr(), 1.0 / M, g.data_ptr(), d.data_ptr(), _ld(d))
            return d

        if chunk >= V:
            # one pass: dlogits for the whole vocabulary (freed after the two products)
            d = dlogits(0, V, padded_empty(M, V, torch.bfloat16, xb.device))
            if ctx.needs_input_grad[0]:
                dX = gemm_raw(d, Wb, "N", "T", out_dtype=ctx.x_dtype)          # dlogits . W^T
            if ctx.needs_input_grad[1]:
                if mg is not None:
                    weight_grad(xb, d, mg)                                       # X^T . dlogits
                else:
                    dW = gemm_raw(xb, d, "T", "N", out_dtype=torch.float32)
            return dX, dW, None
        # vocabulary slices through one reused buffer; dX accumulates in fp32.
        # The slices run on the current stream: a forked product would still be
        # reading the buffer when the next slice overwrites it.
        buf = padded_empty(M, chunk, torch.bfloat16, xb.device)
        dx32 = torch.zeros((M, D), dtype=torch.float32, device=xb.device) if ctx.needs_input_grad[0] else None
        if ctx.needs_input_grad[1]:
            dWt = mg if mg is not None else padded_empty(D, V, torch.float32, xb.device)
        for v0 in range(0, V, chunk):
            vn = min(chunk, V - v0)
            d = dlogits(v0, vn, buf)
            if dx32 is not None:
                gemm_raw(d, Wb[:, v0:v0 + vn], "N", "T", out=dx32, beta=1.0)
            if ctx.needs_input_grad[1]:
                gemm_raw(xb, d, "T", "N", out=dWt[:, v0:v0 + vn])
        if dx32 is not None:
            dX = dx32.to(ctx.x_dtype)
        if ctx.needs_input_grad[1] and mg is None:
            dW = dWt
        return dX, dW, None


def linear_cross_entropy(X: torch.Tensor, W: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    """Mean softmax CE of logits = X[M, D] @ W[D, V] against int targets[M],
    differentiable in X and W, without materialising the (M, V) logits
    (cross_entropy.py:119-124). X is bf16 (leading dims are flattened), W the
    fp32 LM-head weight (its bf16 copy is what the GEMMs read)."""
    if X.dim() < 2 or W.dim() != 2:
        raise ValueError("linear_cross_entropy: X needs >= 2 dims and W exactly 2")
    return _LinearCE.apply(X.reshape(-1, X.shape[-1]), W, targets.reshape(-1))
