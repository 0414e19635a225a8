"""nlearn_amd.kernels.gemm — ``gemm``, ``matmul`` and ``linear`` on the gfx950 MFMA GEMM.

Mirrors nlearn/kernels/gemm.py (same names, same argument meaning):

* ``gemm(A, B)``      differentiable A[M,K] @ B[K,N] -> fp32 C (gemm.py:61-79);
* ``matmul(A, B)``    drop-in for ``@`` on 2-D operands (gemm.py:82-90);
* ``linear(x, W)``    x[..., K] @ W[K, N] as ONE flattened GEMM, output in
                      x's dtype (gemm.py:93-115).

Differences from the reference, all on purpose:

* no host padding: the kernel masks M/N/K tails (gemm.py:47-58 padded to 32/64);
* no materialised transposes in the backward: dA = dC.B^T and dB = A^T.dC are
  the kernel's NT and TN forms (gemm.py:74-75 transposed in XLA);
* ``linear`` writes bf16 straight from the fp32 accumulators (gemm.py:114 wrote
  fp32 then cast), and its weight gradient is produced in fp32 for an fp32
  master weight, so no bf16 rounding of the gradient;
* there is no pure-framework fallback (gemm.py:115): the HIP library is
  required, and a missing library raises.
"""
from __future__ import annotations

import torch

from .. import _lib
from . import wgrad

_BF16 = torch.bfloat16
_F32 = torch.float32


def _check_device(*ts):
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError("nlearn_amd kernels need HIP device tensors (got a CPU tensor)")


def _rows_disjoint(t: torch.Tensor) -> bool:
    """True when no two rows of a 2-D view share memory (row stride >= row
    length). A broadcast view (row stride 0, e.g. the cotangent of a sum over
    rows) is not: the kernels would read or write past its one stored row."""
    return t.shape[0] <= 1 or t.stride(0) >= t.shape[1]


def _ld(t: torch.Tensor) -> int:
    """Leading dimension of a row-major 2-D view (unit column stride, disjoint rows)."""
    if t.dim() != 2:
        raise ValueError(f"expected a 2-D tensor, got shape {tuple(t.shape)}")
    if t.stride(1) != 1 and t.shape[1] > 1:
        raise ValueError("GEMM operands need a unit column stride")
    if not _rows_disjoint(t):
        raise ValueError(f"GEMM operand rows overlap (row stride {t.stride(0)} < row length {t.shape[1]})")
    return t.stride(0) if t.shape[0] > 1 else (t.shape[1] + 7) // 8 * 8


def _aligned(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0 and _ld(t) % 8 == 0


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """bf16, unit column stride, disjoint 16-byte aligned rows; copies only when it must."""
    if t.dtype != _BF16:
        t = t.to(_BF16)
    if t.dim() == 2 and (t.stride(1) == 1 or t.shape[1] <= 1) and _rows_disjoint(t) and _aligned(t):
        return t
    rows, cols = t.shape
    ld = (cols + 7) // 8 * 8
    buf = torch.empty((rows, ld), dtype=_BF16, device=t.device)
    view = buf[:, :cols]
    view.copy_(t)
    return view


def padded_empty(rows: int, cols: int, dtype=_BF16, device="cuda") -> torch.Tensor:
    """A [rows, cols] view whose rows start on 16-byte boundaries (ld rounded to 8).

    Wide rows (>= 1024 columns) are rounded up to 64 elements instead, so every
    row starts on a 128-byte cache line: the GEMM epilogue then writes whole
    lines (the LM-head logits with ld 50264 cost ~30% extra HBM write traffic
    in partial lines, measured with the WRITE_SIZE counter).

    A stride that is a multiple of 1024 elements gets 64 more: with the
    2048-wide FFN activations at ld 2112 instead of 2048 the bs32 x seq512
    training step ran 0.25% faster (A/B over three rounds on one MI355X;
    ld 2176 made no difference)."""
    ld = (cols + 7) // 8 * 8 if cols < 1024 else (cols + 63) // 64 * 64
    if ld >= 1024 and ld % 1024 == 0:
        ld += 64
    return torch.empty((rows, ld), dtype=dtype, device=device)[:, :cols]


EPI_NONE, EPI_BIAS, EPI_BIAS_GELU, EPI_DGELU = 0, 1, 2, 3


def gemm_raw(A: torch.Tensor, B: torch.Tensor, opA: str = "N", opB: str = "N", out_dtype=_F32,
             out: torch.Tensor | None = None, alpha: float = 1.0, beta: float = 0.0,
             alpha_dev: torch.Tensor | None = None, epi: int = EPI_NONE, bias: torch.Tensor | None = None,
             aux: torch.Tensor | None = None, ws: torch.Tensor | None = None) -> torch.Tensor:
    """C = epilogue(alpha * [*alpha_dev] * op(A) @ op(B)) on the current stream.

    opA == "T": A is stored [K, M]; opB == "T": B is stored [N, K].
    epi: EPI_NONE (+ beta * C), EPI_BIAS (+ bias[N] + beta * C), EPI_BIAS_GELU
    (aux = bf16(v + bias), C = gelu_tanh(aux)), EPI_DGELU (C = v * gelu_tanh'(aux)).
    ws: split-K workspace of at least ``gemm_ws_bytes`` bytes (allocated here if None).
    """
    _check_device(A, B)
    A = _kernel_ready(A)
    B = _kernel_ready(B)
    M = A.shape[1] if opA == "T" else A.shape[0]
    K = A.shape[0] if opA == "T" else A.shape[1]
    Kb = B.shape[1] if opB == "T" else B.shape[0]
    N = B.shape[0] if opB == "T" else B.shape[1]
    if K != Kb:
        raise ValueError(f"gemm: inner dimensions differ ({K} vs {Kb})")
    if out is None:
        if beta != 0.0:
            raise ValueError("gemm: beta != 0 needs an output tensor")
        out = padded_empty(M, N, out_dtype, A.device)
    if out.dtype not in (_F32, _BF16):
        raise ValueError("gemm: output must be float32 or bfloat16")
    if tuple(out.shape) != (M, N):
        raise ValueError(f"gemm: output shape {tuple(out.shape)} != {(M, N)}")
    if alpha_dev is not None and (alpha_dev.dtype != _F32 or not alpha_dev.is_cuda):
        raise ValueError("gemm: alpha_dev must be a float32 device scalar")
    if epi in (EPI_BIAS, EPI_BIAS_GELU):
        if bias is None or bias.dtype != _F32 or bias.numel() != N or not bias.is_contiguous():
            raise ValueError("gemm: the bias epilogue needs a contiguous float32 bias of N elements")
    if epi in (EPI_BIAS_GELU, EPI_DGELU):
        if aux is None or aux.dtype != _BF16 or tuple(aux.shape) != (M, N):
            raise ValueError(f"gemm: the GELU epilogues need a bf16 aux of shape {(M, N)}")
    stream = torch.cuda.current_stream(A.device).cuda_stream
    oa = _lib.NL_OP_T if opA == "T" else _lib.NL_OP_N
    ob = _lib.NL_OP_T if opB == "T" else _lib.NL_OP_N
    wsb = int(_lib.load().nl_gemm_ws_bytes(oa, ob, M, N, K))
    if ws is None:
        ws = torch.empty(wsb // 4, dtype=_F32, device=A.device) if wsb else None
    elif ws.numel() * ws.element_size() < wsb:
        raise ValueError("gemm: workspace too small")
    _lib.call("nl_gemm_fused", stream, oa, ob, M, N, K, float(alpha),
              A.data_ptr(), _ld(A), B.data_ptr(), _ld(B), float(beta), out.data_ptr(),
              _lib.NL_DTYPE_F32 if out.dtype == _F32 else _lib.NL_DTYPE_BF16, _ld(out),
              alpha_dev.data_ptr() if alpha_dev is not None else None, int(epi),
              bias.data_ptr() if bias is not None else None,
              aux.data_ptr() if aux is not None else None, _ld(aux) if aux is not None else 0,
              ws.data_ptr() if ws is not None else None, wsb)
    return out


def gemm_ws(opA: str, opB: str, M: int, N: int, K: int, device) -> torch.Tensor | None:
    """The split-K workspace gemm_raw would allocate for this product (or None)."""
    oa = _lib.NL_OP_T if opA == "T" else _lib.NL_OP_N
    ob = _lib.NL_OP_T if opB == "T" else _lib.NL_OP_N
    wsb = int(_lib.load().nl_gemm_ws_bytes(oa, ob, M, N, K))
    return torch.empty(wsb // 4, dtype=_F32, device=device) if wsb else None


def weight_grad(X: torch.Tensor, dY: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out = X^T . dY (fp32), forked onto the weight-gradient stream when one is
    active (nlearn_amd.kernels.wgrad); operands and workspace are prepared on
    the current stream first, so the forked kernels allocate nothing."""
    X = _kernel_ready(X)
    dY = _kernel_ready(dY)
    ws = gemm_ws("T", "N", X.shape[1], dY.shape[1], X.shape[0], X.device)
    wgrad.fork(lambda: gemm_raw(X, dY, "T", "N", out=out, ws=ws), X, dY, out, ws)
    return out


# ---------------------------------------------------------------------------
# bf16 shadows of fp32 weights (model.py:372-375 casts every parameter each step)
# ---------------------------------------------------------------------------


def bf16_shadow(W: torch.Tensor) -> torch.Tensor:
    """The bf16 copy of an fp32 weight, refreshed only when the weight changed.

    An optimizer that writes the bf16 copy itself (the fused AdamW) tags it with
    the weight's version counter so this returns it without another cast.
    """
    if W.dtype == _BF16:
        return W
    sh = getattr(W, "_nl_bf16", None)
    if sh is not None and getattr(W, "_nl_bf16_version", None) == W._version:
        return sh
    sh = _kernel_ready(W.detach())
    if sh.data_ptr() == W.data_ptr():  # pragma: no cover - dtype differs, cannot alias
        sh = sh.clone()
    W._nl_bf16 = sh
    W._nl_bf16_version = W._version
    return sh


def grad_buffer(W: torch.Tensor) -> torch.Tensor | None:
    """W's preallocated fp32 gradient buffer (``W.main_grad``), or None.

    The optimizer attaches these once (fixed addresses, so a captured step
    writes the same memory every replay); a backward that finds one writes the
    weight gradient straight into it and returns no gradient to autograd."""
    return getattr(W, "main_grad", None)


# ---------------------------------------------------------------------------
# gemm — gemm.py:61-79
# ---------------------------------------------------------------------------


class _Gemm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, A, B):
        ctx.save_for_backward(A, B)
        return gemm_raw(A, B, out_dtype=_F32)

    @staticmethod
    def backward(ctx, dC):
        A, B = ctx.saved_tensors
        dA = dB = None
        if ctx.needs_input_grad[0]:
            dA = gemm_raw(dC, B, "N", "T", out_dtype=_F32).to(A.dtype)   # dC . B^T
        if ctx.needs_input_grad[1]:
            dB = gemm_raw(A, dC, "T", "N", out_dtype=_F32).to(B.dtype)   # A^T . dC
        return dA, dB


def gemm(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """Differentiable A[M,K] @ B[K,N] -> C[M,N] (fp32), bf16 operands."""
    return _Gemm.apply(A, B)


def matmul(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """``A @ B`` on the HIP GEMM. 2-D x 2-D is one kernel; a leading batch of A
    ([..., M, K] @ [K, N]) is flattened into M. Other shapes are rejected."""
    if A.dim() == 2 and B.dim() == 2:
        return gemm(A, B)
    if A.dim() > 2 and B.dim() == 2:
        lead = A.shape[:-1]
        return gemm(A.reshape(-1, A.shape[-1]), B).reshape(*lead, B.shape[1])
    raise ValueError(f"matmul: unsupported operand ranks {A.dim()} and {B.dim()}")


# ---------------------------------------------------------------------------
# linear — gemm.py:93-115
# ---------------------------------------------------------------------------


def linear_backward(x2, W, Wb, dy, need_dx: bool = True, need_dW: bool = True):
    """(dX, dW) of Y = X . W from dY: dX = dY . W^T on the current stream, dW =
    X^T . dY into W's gradient buffer (forked onto the weight-gradient stream
    when one is active; dW is then None) or returned."""
    dx = dW = None
    if need_dx:
        dx = gemm_raw(dy, Wb, "N", "T", out_dtype=x2.dtype)             # dY . W^T
    if need_dW:
        mg = grad_buffer(W)
        if mg is not None:
            weight_grad(x2, dy, mg)                                            # X^T . dY -> main_grad
        else:
            dW = gemm_raw(x2, dy, "T", "N", out_dtype=_F32 if W.dtype == _F32 else W.dtype)
    return dx, dW


class _Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x2, W):
        Wb = bf16_shadow(W)
        out_dtype = x2.dtype if x2.dtype in (_BF16, _F32) else _F32
        y = gemm_raw(x2, Wb, out_dtype=out_dtype)
        ctx.save_for_backward(x2, W)
        ctx.wb = Wb
        return y

    @staticmethod
    def backward(ctx, dy):
        x2, W = ctx.saved_tensors
        return linear_backward(x2, W, ctx.wb, dy, ctx.needs_input_grad[0], ctx.needs_input_grad[1])


def linear(x: torch.Tensor, W: torch.Tensor) -> torch.Tensor:
    """x[..., K] @ W[K, N] -> [..., N] in x's dtype, as one GEMM with M = prod(lead)."""
    if x.dim() < 2 or W.dim() != 2:
        raise ValueError("linear: x needs >= 2 dims and W exactly 2")
    lead = x.shape[:-1]
    y = _Linear.apply(x.reshape(-1, x.shape[-1]), W)
    return y.reshape(*lead, W.shape[1])
