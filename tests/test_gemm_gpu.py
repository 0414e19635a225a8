"""GPU parity of the MFMA GEMM (NN forward, NT dX, TN dW) against the oracle.

Tolerance (north_star): relative L2 <= 5e-3 (fp32 accumulation); integer-valued
inputs whose partial sums stay below 2^24 must match exactly.
"""
import numpy as np
import pytest

from conftest import GOLDEN, rel_l2
from oracle import ops

pytestmark = pytest.mark.gpu


def _dev_bf16(a, dev):
    import torch

    bits = ops.bf16_bits(a) if a.dtype != np.uint16 else a
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)


def _np(t):
    import torch

    if t.dtype == torch.bfloat16:
        return ops.bf16_to_f32(t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))
    return t.contiguous().cpu().numpy()


@pytest.mark.parametrize("name", ["gemm_small", "gemm_medium", "gemm_large_magnitude"])
def test_gemm_golden(dev, name):
    import torch
    from nlearn_amd.kernels.gemm import gemm_raw

    g = np.load(GOLDEN / f"{name}.npz")
    C = gemm_raw(_dev_bf16(g["A"], dev), _dev_bf16(g["B"], dev))
    torch.cuda.synchronize()
    assert rel_l2(_np(C), g["C"]) <= 5e-3


@pytest.mark.parametrize("opA,opB", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (7, 9, 13), (32, 32, 16), (100, 130, 70), (257, 255, 129),
                                   (300, 520, 1000), (64, 50257, 64), (513, 200, 50257)])
def test_gemm_layouts_exact_small_integers(dev, opA, opB, M, N, K):
    """Small integers: every product and partial sum is exact in fp32."""
    import torch
    from nlearn_amd.kernels.gemm import gemm_raw

    rng = np.random.default_rng(M + 7 * N + 13 * K)
    A = rng.integers(-3, 4, (M, K)).astype(np.float32)
    B = rng.integers(-3, 4, (K, N)).astype(np.float32)
    As = A.T.copy() if opA == "T" else A
    Bs = B.T.copy() if opB == "T" else B
    ref = ops.gemm(As, Bs, opA, opB)
    C = gemm_raw(_dev_bf16(As, dev), _dev_bf16(Bs, dev), opA, opB)
    torch.cuda.synchronize()
    assert np.array_equal(_np(C), ref)


@pytest.mark.parametrize("opA,opB", [("N", "N"), ("N", "T"), ("T", "N")])
def test_gemm_bf16_out_alpha_beta_and_device_scale(dev, opA, opB):
    import torch
    from nlearn_amd.kernels.gemm import gemm_raw, padded_empty

    rng = np.random.default_rng(11)
    M, N, K = 300, 200, 96
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    As = A.T.copy() if opA == "T" else A
    Bs = B.T.copy() if opB == "T" else B
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    out = padded_empty(M, N, torch.float32, dev)
    out.copy_(torch.from_numpy(C0))
    s = torch.tensor(0.5, device=dev)
    gemm_raw(_dev_bf16(As, dev), _dev_bf16(Bs, dev), opA, opB, out=out, alpha=2.0, beta=-1.0, alpha_dev=s)
    ref = 1.0 * ops.gemm(As, Bs, opA, opB) - C0
    torch.cuda.synchronize()
    assert rel_l2(_np(out), ref) <= 5e-3
    ob = gemm_raw(_dev_bf16(As, dev), _dev_bf16(Bs, dev), opA, opB, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert rel_l2(_np(ob), ops.gemm(As, Bs, opA, opB)) <= 5e-3


@pytest.mark.parametrize("K,N", [(512, 1536), (512, 512), (512, 2048), (2048, 512), (512, 50257)])
def test_gemm_model_shapes(dev, K, N):
    """M = 16384 (bs32 x seq512): forward, dX = dY W^T and dW = X^T dY, checked on
    sampled rows / columns against the float64 oracle."""
    import torch
    from nlearn_amd.kernels.gemm import gemm_raw, padded_empty

    M = 16384
    gen = torch.Generator(device=dev).manual_seed(K + N)
    X = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
    W = padded_empty(K, N, torch.bfloat16, dev)
    W.copy_(torch.randn((K, N), generator=gen, device=dev) * 0.02)
    dY = padded_empty(M, N, torch.bfloat16, dev)
    dY.copy_(torch.randn((M, N), generator=gen, device=dev))
    Y = gemm_raw(X, W, out_dtype=torch.bfloat16)
    dX = gemm_raw(dY, W, "N", "T", out_dtype=torch.bfloat16)
    dW = gemm_raw(X, dY, "T", "N", out_dtype=torch.float32)
    torch.cuda.synchronize()
    rng = np.random.default_rng(0)
    rows = rng.choice(M, 48, replace=False)
    cols = rng.choice(N, 48, replace=False)
    Xn, Wn = _np(X), _np(W)
    rows_t = torch.from_numpy(rows).to(dev)
    cols_t = torch.from_numpy(cols).to(dev)
    assert rel_l2(_np(Y[rows_t]), ops.gemm(Xn[rows], Wn)) <= 5e-3
    assert rel_l2(_np(dX[rows_t]), ops.gemm(_np(dY[rows_t]), Wn, "N", "T")) <= 5e-3
    assert rel_l2(_np(dW[:, cols_t]), ops.gemm(Xn, _np(dY[:, cols_t]), "T", "N")) <= 5e-3


def test_linear_autograd(dev):
    import torch
    from nlearn_amd.kernels.gemm import linear

    rng = np.random.default_rng(5)
    x = torch.from_numpy(ops.bf16_round(rng.standard_normal((4, 33, 64)).astype(np.float32))).to(dev)
    W = torch.from_numpy((rng.standard_normal((64, 72)) * 0.1).astype(np.float32)).to(dev)
    xb = x.to(torch.bfloat16).requires_grad_(True)
    Wp = W.clone().requires_grad_(True)
    y = linear(xb, Wp)
    assert y.dtype == torch.bfloat16 and y.shape == (4, 33, 72)
    gy = torch.from_numpy(ops.bf16_round(rng.standard_normal((4, 33, 72)).astype(np.float32))).to(dev)
    y.backward(gy.to(torch.bfloat16))
    xn, Wn, gn = x.cpu().numpy().reshape(-1, 64), W.cpu().numpy(), gy.cpu().numpy().reshape(-1, 72)
    assert rel_l2(_np(y).reshape(-1, 72), ops.gemm(xn, Wn)) <= 5e-3
    assert rel_l2(_np(xb.grad).reshape(-1, 64), ops.gemm(gn, Wn, "N", "T")) <= 5e-3
    assert Wp.grad.dtype == torch.float32
    assert rel_l2(Wp.grad.cpu().numpy(), ops.gemm(xn, gn, "T", "N")) <= 5e-3


@pytest.mark.parametrize("M,N,K", [(512, 512, 16384), (2048, 512, 16384), (512, 1536, 4096), (100, 70, 5000)])
def test_gemm_split_k_matches_single_pass_and_is_deterministic(dev, M, N, K):
    """Weight-gradient shapes (small output, long reduction) take the split-K
    path when a workspace is given; it must agree with the one-pass kernel and
    give bitwise-identical results run to run."""
    import torch
    from nlearn_amd import _lib
    from nlearn_amd.kernels.gemm import gemm_raw, padded_empty

    gen = torch.Generator(device=dev).manual_seed(M + N + K)
    X = padded_empty(K, M, torch.bfloat16, dev)   # A stored [K][M] (opA = T)
    X.copy_(torch.randn((K, M), generator=gen, device=dev))
    dY = padded_empty(K, N, torch.bfloat16, dev)
    dY.copy_(torch.randn((K, N), generator=gen, device=dev))
    assert _lib.load().nl_gemm_ws_bytes(1, 0, M, N, K) > 0
    split1 = gemm_raw(X, dY, "T", "N", out_dtype=torch.float32)
    split2 = gemm_raw(X, dY, "T", "N", out_dtype=torch.float32)
    single = padded_empty(M, N, torch.float32, dev)
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("nl_gemm", st, 1, 0, M, N, K, 1.0, X.data_ptr(), X.stride(0), dY.data_ptr(), dY.stride(0), 0.0,
              single.data_ptr(), 0, single.stride(0), None)
    torch.cuda.synchronize()
    assert torch.equal(split1, split2)
    assert rel_l2(_np(split1), _np(single)) <= 1e-5
    cols = np.random.default_rng(1).choice(N, min(N, 32), replace=False)
    ct = torch.from_numpy(cols).to(dev)
    assert rel_l2(_np(split1[:, ct]), ops.gemm(_np(X), _np(dY[:, ct]), "T", "N")) <= 5e-3


def test_gemm_ex_workspace_contract(dev):
    """nl_gemm_ex splits K only when the workspace holds nl_gemm_ws_bytes: one
    byte less (or none) gives the one-pass result, bit for bit that of nl_gemm;
    the full size gives the split result, bit for bit that of gemm_raw."""
    import torch
    from nlearn_amd import _lib
    from nlearn_amd.kernels.gemm import gemm_raw, padded_empty

    M, N, K = 512, 1536, 16384
    gen = torch.Generator(device=dev).manual_seed(21)
    X = padded_empty(K, M, torch.bfloat16, dev)
    X.copy_(torch.randn((K, M), generator=gen, device=dev))
    dY = padded_empty(K, N, torch.bfloat16, dev)
    dY.copy_(torch.randn((K, N), generator=gen, device=dev))
    need = int(_lib.load().nl_gemm_ws_bytes(1, 0, M, N, K))
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    outs = {}
    for name, wsb in (("none", 0), ("short", need - 1), ("full", need)):
        c = padded_empty(M, N, torch.float32, dev)
        _lib.call("nl_gemm_ex", st, 1, 0, M, N, K, 1.0, X.data_ptr(), X.stride(0), dY.data_ptr(), dY.stride(0), 0.0,
                  c.data_ptr(), 0, c.stride(0), None, ws.data_ptr() if wsb else None, wsb)
        outs[name] = c
    single = padded_empty(M, N, torch.float32, dev)
    _lib.call("nl_gemm", st, 1, 0, M, N, K, 1.0, X.data_ptr(), X.stride(0), dY.data_ptr(), dY.stride(0), 0.0,
              single.data_ptr(), 0, single.stride(0), None)
    split = gemm_raw(X, dY, "T", "N", out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(outs["none"], single)
    assert torch.equal(outs["short"], single)
    assert torch.equal(outs["full"], split)
    assert rel_l2(_np(outs["full"]), _np(single)) <= 1e-5


@pytest.mark.parametrize("opA,opB,M,N,K,out", [("N", "N", 2000, 9000, 3000, "f32"), ("N", "T", 4000, 600, 25000, "f32"),
                                                ("T", "N", 600, 9000, 10000, "f32"), ("N", "N", 2000, 9000, 3000, "bf16"),
                                                ("N", "N", 4000, 12000, 1152, "bf16"), ("N", "N", 4000, 12000, 1152, "f32"),
                                                ("N", "T", 4000, 12000, 1152, "bf16"), ("T", "N", 4000, 12000, 1152, "f32")])
def test_gemm_huge_tile_path_exact_small_integers(dev, opA, opB, M, N, K, out):
    """Products of >= 100 GFLOP take the 256 x 256 tile path (8 waves; split K
    for short grids: NT here splits 5 ways, TN 2 ways). With K % 128 == 0,
    K <= 4096 and no split (the 1152-deep cases) the persistent variant runs:
    one workgroup per CU over many tiles, interior and edge tiles mixed.
    Ragged M, N and K (a masked k tail), checked exactly on integer inputs
    (every partial sum is an integer below 2^24, so fp32 accumulation is exact
    in any order and bf16 output is the single rounding of the exact value)."""
    import torch
    from nlearn_amd.kernels.gemm import gemm_raw

    assert 2.0 * M * N * K >= 1e11                      # the dispatcher picks the 256 x 256 tiles
    rng = np.random.default_rng(M + N + K)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    As = A.T.copy() if opA == "T" else A
    Bs = B.T.copy() if opB == "T" else B
    dt = torch.float32 if out == "f32" else torch.bfloat16
    C = gemm_raw(_dev_bf16(As, dev), _dev_bf16(Bs, dev), opA, opB, out_dtype=dt)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(0, 260), np.arange(M - 260, M), rng.integers(0, M, 100)]))
    got = C[torch.from_numpy(rows).to(dev)].float().cpu().numpy()
    ref = A[rows] @ B
    if out == "bf16":
        ref = torch.from_numpy(ref).bfloat16().float().numpy()
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("opA,M,N,K", [("T", 500, 50257, 200), ("N", 16312, 8192, 72)])
def test_gemm_tall_tile_path_exact_small_integers(dev, opA, M, N, K):
    """Products large enough for the 256 x 128 tile path (ragged M, N and K),
    checked exactly on integer inputs over sampled rows including both edges."""
    import torch
    from nlearn_amd import _lib
    from nlearn_amd.kernels.gemm import gemm_raw

    tiles128 = ((M + 127) // 128) * ((N + 127) // 128)
    assert tiles128 >= (1024 if opA == "T" else 8192)       # the dispatcher picks the tall tiles
    rng = np.random.default_rng(M + N + K)
    A = rng.integers(-3, 4, (M, K)).astype(np.float32)
    B = rng.integers(-3, 4, (K, N)).astype(np.float32)
    As = A.T.copy() if opA == "T" else A
    C = gemm_raw(_dev_bf16(As, dev), _dev_bf16(B, dev), opA, "N")
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(0, 130), np.arange(M - 130, M), rng.integers(0, M, 200)]))
    got = C[torch.from_numpy(rows).to(dev)].float().cpu().numpy()
    assert np.array_equal(got, A[rows] @ B)


@pytest.mark.parametrize("opB,M,N,K,out", [("N", 4100, 4000, 128, "f32"), ("N", 4100, 4000, 256, "bf16"),
                                           ("T", 4097, 4033, 384, "f32"), ("T", 16384, 2048, 512, "bf16"),
                                           ("N", 16384, 1536, 512, "bf16")])
def test_gemm_persistent_128_path_exact_small_integers(dev, opB, M, N, K, out):
    """Short-K NN / NT products without an epilogue and with at least 4 tiles
    of 128 x 128 per workgroup (two per CU) run the persistent 128 x 128
    kernel: interior and ragged edge tiles, fp32 and bf16 outputs, checked
    exactly on integer inputs over sampled rows including both edges."""
    import torch
    from nlearn_amd.kernels.gemm import gemm_raw

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    assert K % 128 == 0 and ((M + 127) // 128) * ((N + 127) // 128) >= 4 * cus
    rng = np.random.default_rng(M + N + K)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    Bs = B.T.copy() if opB == "T" else B
    dt = torch.float32 if out == "f32" else torch.bfloat16
    C = gemm_raw(_dev_bf16(A, dev), _dev_bf16(Bs, dev), "N", opB, out_dtype=dt)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(0, 130), np.arange(M - 130, M), rng.integers(0, M, 200)]))
    got = C[torch.from_numpy(rows).to(dev)].float().cpu().numpy()
    ref = A[rows] @ B
    if out == "bf16":
        ref = torch.from_numpy(ref).bfloat16().float().numpy()
    assert np.array_equal(got, ref)


def test_persistent_gemm_beside_inplace_ce_on_another_stream(dev):
    """Regression: the persistent GEMM kernel's raw barriers once let a wave
    pass with LDS fragment reads still pending, so another wave's DMA into the
    same stage buffer could overwrite them. It showed as wrong 32- to 128-column
    blocks of the output when an in-place CE ran beside the GEMM on another
    stream (the LM head + CE in two chunks at 3000 rows: CE of rows [0, 1792)
    beside the persistent 128 x 128 GEMM of rows [1792, 3000)). The GEMM beside
    the CE must equal the GEMM alone, bit for bit, every time."""
    import torch
    from nlearn_amd import _lib
    from nlearn_amd.kernels import wgrad
    from nlearn_amd.kernels.gemm import _ld, bf16_shadow, gemm_raw, padded_empty

    M, V, cut = 3000, 50257, 1792
    rng = np.random.default_rng(3)
    X = torch.from_numpy(rng.standard_normal((M, 512)).astype(np.float32) * 0.5).to(dev).bfloat16()
    W = torch.from_numpy(rng.standard_normal((512, V)).astype(np.float32) * 0.05).to(dev)
    t = torch.from_numpy(rng.integers(0, V, M).astype(np.int32)).to(dev)
    Wb = bf16_shadow(W)
    alone = gemm_raw(X[cut:], Wb, out=padded_empty(M - cut, V, torch.bfloat16, dev))
    main, aux = torch.cuda.current_stream(), wgrad._side_stream(dev, 1)
    for _ in range(4):
        logits = padded_empty(M, V, torch.bfloat16, dev)
        loss, lse = torch.empty(M, device=dev), torch.empty(M, device=dev)
        gemm_raw(X[:cut], Wb, out=logits[:cut])
        aux.wait_stream(main)
        with torch.cuda.stream(aux):
            _lib.call("nl_ce_fwd_bwd", aux.cuda_stream, cut, V, logits.data_ptr(), _ld(logits), t.data_ptr(),
                      loss.data_ptr(), lse.data_ptr(), 1.0 / M, logits.data_ptr(), _ld(logits))
        gemm_raw(X[cut:], Wb, out=logits[cut:])
        main.wait_stream(aux)
        torch.cuda.synchronize()
        assert torch.equal(logits[cut:], alone)
