"""The reference-named GEMM wrappers and the GEMM's reach beyond 2 GB operands.

* ``gemm(A, B)`` (gemm.py:61-79) forward and autograd, and ``matmul`` on 2-D
  and batched-lead operands (gemm.py:82-90), against the float64 oracle
  (tolerance rel-L2 <= 5e-3, north_star's GEMM bar).
* ``linear``'s backward with a broadcast cotangent (row stride 0), against a
  float64 reference of the same products.
* Products whose operands span 2 GB or more: the library cuts them into
  sub-products (panels of M or N, chunks of K) that fit 32-bit buffer offsets.
  Each of the four cases runs on small-integer data, where every partial sum
  is exact in fp32, and is checked exactly on sampled rows or columns,
  including the rows next to the panel boundaries.
"""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import ops

pytestmark = pytest.mark.gpu
TOL = 5e-3


def _np(t):
    import torch

    if t.dtype == torch.bfloat16:
        return ops.bf16_to_f32(t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))
    return t.detach().contiguous().cpu().numpy()


def _bf16(a, dev, requires_grad=False):
    import torch

    t = torch.from_numpy(ops.bf16_round(np.asarray(a, np.float32))).to(dev).to(torch.bfloat16)
    return t.requires_grad_(requires_grad)


def test_gemm_autograd_matches_oracle(dev):
    import torch
    from nlearn_amd.kernels.gemm import gemm

    rng = np.random.default_rng(61)
    M, K, N = 300, 200, 170
    A = ops.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    B = ops.bf16_round((rng.standard_normal((K, N)) * 0.02).astype(np.float32))
    dC = ops.bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    a, b = _bf16(A, dev, True), _bf16(B, dev, True)
    c = gemm(a, b)
    assert c.dtype == torch.float32 and tuple(c.shape) == (M, N)
    c.backward(torch.from_numpy(dC).to(dev))
    torch.cuda.synchronize()
    assert rel_l2(_np(c), ops.gemm(A, B)) <= TOL
    # dA = dC . B^T and dB = A^T . dC (gemm.py:74-75), returned in the operands' dtype
    assert a.grad.dtype == torch.bfloat16 and b.grad.dtype == torch.bfloat16
    assert rel_l2(_np(a.grad), ops.gemm(dC, B, "N", "T")) <= TOL
    assert rel_l2(_np(b.grad), ops.gemm(A, dC, "T", "N")) <= TOL


def test_matmul_2d_and_batched_lead(dev):
    import torch
    from nlearn_amd.kernels.gemm import matmul

    rng = np.random.default_rng(62)
    A2 = rng.standard_normal((77, 96)).astype(np.float32)
    A3 = rng.standard_normal((3, 41, 96)).astype(np.float32)
    B = rng.standard_normal((96, 130)).astype(np.float32)
    b = _bf16(B, dev)
    c2 = matmul(_bf16(A2, dev), b)
    c3 = matmul(_bf16(A3, dev), b)
    torch.cuda.synchronize()
    assert tuple(c3.shape) == (3, 41, 130)
    assert rel_l2(_np(c2), ops.gemm(ops.bf16_round(A2), ops.bf16_round(B))) <= TOL
    ref3 = ops.gemm(ops.bf16_round(A3.reshape(-1, 96)), ops.bf16_round(B)).reshape(3, 41, 130)
    assert rel_l2(_np(c3), ref3) <= TOL
    with pytest.raises(ValueError):
        matmul(_bf16(B, dev), _bf16(A3, dev))


def test_linear_backward_with_broadcast_cotangent(dev):
    """(linear(x, W).sum(0) * w).sum() in bf16 hands the backward a bf16
    cotangent whose rows all alias one stored row (strides (0, 1)); dX and dW
    must be those of the materialised cotangent."""
    import torch
    from nlearn_amd.kernels import gemm as G

    rng = np.random.default_rng(63)
    M, K, N = 256, 128, 96
    X = ops.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    W = (rng.standard_normal((K, N)) * 0.05).astype(np.float32)
    w = ops.bf16_round(rng.standard_normal(N).astype(np.float32))
    x = _bf16(X, dev, True)
    Wd = torch.from_numpy(W).to(dev).requires_grad_(True)
    seen = []
    orig = G._kernel_ready

    def spy(t):
        seen.append(tuple(t.stride()))
        return orig(t)

    G._kernel_ready = spy
    try:
        y = G.linear(x, Wd)
        (y.sum(0) * _bf16(w, dev)).sum().backward()
    finally:
        G._kernel_ready = orig
    torch.cuda.synchronize()
    assert (0, 1) in seen          # the broadcast cotangent did reach the GEMM wrapper
    dY = np.broadcast_to(w, (M, N))
    assert rel_l2(_np(x.grad), ops.gemm(dY, ops.bf16_round(W), "N", "T")) <= TOL
    assert rel_l2(_np(Wd.grad), ops.gemm(X, dY, "T", "N")) <= TOL


# ---------------------------------------------------------------------------
# operands of 2 GB and more
# ---------------------------------------------------------------------------

BIG_ROWS, BIG_COLS, BIG_LD = 32768, 50257, 50304     # 3.3 GB of bf16: dlogits at bs64 x seq512


@pytest.fixture(scope="module")
def big(dev):
    """A (32768, 50257) bf16 matrix of integers in [-2, 2] with row stride
    50304; the 47 padding columns hold NaN (never part of a product)."""
    import torch

    g = torch.Generator(device=dev).manual_seed(2048)
    base = torch.full((BIG_ROWS, BIG_LD), float("nan"), dtype=torch.bfloat16, device=dev)
    view = base[:, :BIG_COLS]
    for r0 in range(0, BIG_ROWS, 4096):
        view[r0:r0 + 4096].copy_(torch.randint(-2, 3, (4096, BIG_COLS), dtype=torch.int8, device=dev, generator=g))
    torch.cuda.synchronize()
    yield view
    del base, view
    torch.cuda.empty_cache()


def _ints(rng, shape, dev, ld=None):
    """Integer matrix in [-2, 2] as a bf16 device view (row stride ld) and float64 host copy."""
    import torch

    a = rng.integers(-2, 3, shape).astype(np.float32)
    ld = ld or shape[1]
    base = torch.zeros((shape[0], ld), dtype=torch.bfloat16, device=dev)
    base[:, :shape[1]] = torch.from_numpy(a).to(dev)
    return base[:, :shape[1]], a.astype(np.float64)


def _rows_of(view, idx):
    import torch

    return view[torch.as_tensor(idx, device=view.device)].float().cpu().numpy().astype(np.float64)


def _cols_of(view, idx):
    import torch

    return view[:, torch.as_tensor(idx, device=view.device)].float().cpu().numpy().astype(np.float64)


EDGE = [0, 1, 255, 256, 16383, 16384, 16385, 20991, 20992, 21087, 21088, 32511, 32767]


def test_gemm_nt_m_panels_beyond_2gb(dev, big):
    """dX = dlogits . W^T at bs64: A is 3.3 GB k-contiguous -> panels of M."""
    import torch
    from nlearn_amd.kernels.gemm import gemm_raw

    rng = np.random.default_rng(71)
    W, Wh = _ints(rng, (512, BIG_COLS), dev, ld=50264)          # stored [N][K]
    print("gemm NT M-panels 32768x512x50257", flush=True)
    C = gemm_raw(big, W, "N", "T")
    torch.cuda.synchronize()
    rows = sorted(set(EDGE) | set(rng.integers(0, BIG_ROWS, 12).tolist()))
    ref = _rows_of(big, rows) @ Wh.T
    assert np.array_equal(_np(C)[rows].astype(np.float64), ref)


@pytest.mark.parametrize("bias", [False, True])
def test_gemm_tn_k_chunks_beyond_2gb(dev, big, bias):
    """dW = X^T . dlogits at bs64: B is 3.3 GB k-strided -> chunks of K summed
    into the fp32 output (the bias is added once)."""
    import torch
    from nlearn_amd.kernels.gemm import EPI_BIAS, EPI_NONE, gemm_raw

    rng = np.random.default_rng(72)
    X, Xh = _ints(rng, (BIG_ROWS, 512), dev)                    # stored [K][M]
    b = rng.integers(-3, 4, BIG_COLS).astype(np.float32) if bias else None
    print(f"gemm TN K-chunks 512x50257x32768 bias={bias}", flush=True)
    C = gemm_raw(X, big, "T", "N", epi=EPI_BIAS if bias else EPI_NONE,
                 bias=torch.from_numpy(b).to(dev) if bias else None)
    torch.cuda.synchronize()
    cols = sorted(set([0, 1, 255, 256, 50255, 50256]) | set(rng.integers(0, BIG_COLS, 12).tolist()))
    ref = Xh.T @ _cols_of(big, cols)
    if bias:
        ref = ref + b[cols].astype(np.float64)
    assert np.array_equal(_np(C)[:, cols].astype(np.float64), ref)


def test_gemm_nn_k_chunks_beyond_2gb_and_bf16_refusal(dev, big):
    """A k-strided B of 3.3 GB in the forward form: chunks of K; a bf16 C
    cannot carry the running sum, so that request is refused."""
    import torch
    from nlearn_amd import _lib
    from nlearn_amd.kernels.gemm import gemm_raw

    rng = np.random.default_rng(73)
    A, Ah = _ints(rng, (128, BIG_ROWS), dev)
    print("gemm NN K-chunks 128x50257x32768", flush=True)
    C = gemm_raw(A, big, "N", "N")
    torch.cuda.synchronize()
    cols = sorted(set([0, 7, 50000, 50256]) | set(rng.integers(0, BIG_COLS, 12).tolist()))
    assert np.array_equal(_np(C)[:, cols].astype(np.float64), Ah @ _cols_of(big, cols))
    with pytest.raises(_lib.NlError, match="fp32"):
        gemm_raw(A, big, "N", "N", out_dtype=torch.bfloat16)


def test_gemm_nt_n_panels_beyond_2gb(dev, big):
    """A k-contiguous B of 3.3 GB (opB = T): panels of N."""
    import torch
    from nlearn_amd.kernels.gemm import gemm_raw

    rng = np.random.default_rng(74)
    A, Ah = _ints(rng, (256, BIG_COLS), dev, ld=50264)
    print("gemm NT N-panels 256x32768x50257", flush=True)
    C = gemm_raw(A, big, "N", "T")
    torch.cuda.synchronize()
    cols = sorted(set(EDGE) | set(rng.integers(0, BIG_ROWS, 12).tolist()))
    ref = Ah @ _rows_of(big, cols).T
    assert np.array_equal(_np(C)[:, cols].astype(np.float64), ref)


@pytest.mark.parametrize("epi", ["none", "bias", "bias_gelu"])
def test_gemm_k_zero_large_output(dev, epi):
    """K = 0 with null A and B over an output of more than 1024 tiles of
    128 x 128 (the size the persistent short-K kernel takes for K >= 128):
    C = epilogue(0), with no operand read."""
    import torch
    from nlearn_amd import _lib
    from nlearn_amd.kernels.gemm import EPI_BIAS, EPI_BIAS_GELU, EPI_NONE
    from oracle import model_np as om

    M, N = 4100, 4000
    C = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=dev)
    bias = torch.arange(N, dtype=torch.float32, device=dev) / 8
    aux = torch.full((M, N), 5.0, dtype=torch.bfloat16, device=dev)
    code = {"none": EPI_NONE, "bias": EPI_BIAS, "bias_gelu": EPI_BIAS_GELU}[epi]
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("nl_gemm_fused", st, _lib.NL_OP_N, _lib.NL_OP_N, M, N, 0, 1.0, None, 8, None, N, 0.0,
              C.data_ptr(), _lib.NL_DTYPE_BF16, N, None, code,
              bias.data_ptr() if epi != "none" else None, aux.data_ptr() if epi == "bias_gelu" else None,
              N if epi == "bias_gelu" else 0, None, 0)
    torch.cuda.synchronize()
    if epi == "none":
        assert torch.count_nonzero(C).item() == 0
        return
    u = bias.to(torch.bfloat16).expand(M, N)
    if epi == "bias":
        assert torch.equal(C, u)
    else:
        assert torch.equal(aux, u)
        ref = om._gelu(_np(u).astype(np.float64))[0]
        assert np.abs(_np(C) - ref).max() <= np.abs(ref).max() * 2 ** -8 + 1e-6
