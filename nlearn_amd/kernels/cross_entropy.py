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
"""
from __future__ import annotations

import torch

from .. import _lib
from .gemm import _check_device

_BF16 = torch.bfloat16


def _as_rows(logits: torch.Tensor) -> torch.Tensor:
    V = logits.shape[-1]
    x = logits.reshape(-1, V)
    if x.stride(-1) != 1:
        raise ValueError("cross_entropy: logits need a unit stride along the vocabulary")
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
