"""GPU parity of the fused non-GEMM kernels and GEMM epilogues against the oracle.

* LayerNorm forward: the residual sum is bit-exact (one fp32 add, one RNE);
  y within bf16 rounding (rel L2 <= 4e-3); statistics rel 1e-5.
* LayerNorm backward: dx rel L2 <= 1e-2 (bf16 output), dgamma / dbeta rel L2
  <= 1e-4, bitwise reproducible run to run.
* Column sums and the position-embedding gradient: integer-valued inputs make
  every partial sum exact, so the result must match bit for bit.
* GEMM epilogues: integer-valued operands make op(A).op(B) + bias exact, so the
  saved pre-activation is bit-exact; gelu / gelu' outputs within bf16 rounding.
* Embedding forward: bit-exact (fp32 add, one RNE); invalid ids give NaN rows.
"""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import model_np as om
from oracle import ops

pytestmark = pytest.mark.gpu


def _dev_bf16(a, dev):
    import torch

    bits = ops.bf16_bits(a)
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)


def _np(t):
    import torch

    if t.dtype == torch.bfloat16:
        return ops.bf16_to_f32(t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))
    return t.detach().contiguous().cpu().numpy()


def _f32(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


# ---------------------------------------------------------------------------
# LayerNorm
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("rows,D", [(1, 8), (3, 64), (257, 512), (64, 768), (33, 1024), (5, 4096), (16384, 512)])
@pytest.mark.parametrize("residual", [False, True])
def test_layernorm_fwd_bwd(dev, rows, D, residual):
    import torch
    from nlearn_amd.kernels.fused import layer_norm_bwd_raw, layer_norm_fwd_raw

    rng = np.random.default_rng(rows * 31 + D + residual)
    x = ops.bf16_round(rng.standard_normal((rows, D)).astype(np.float32) * 2 + 0.5)
    r = ops.bf16_round(rng.standard_normal((rows, D)).astype(np.float32))
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    b = (0.1 * rng.standard_normal(D)).astype(np.float32)
    dy = ops.bf16_round(rng.standard_normal((rows, D)).astype(np.float32))
    dres = ops.bf16_round(rng.standard_normal((rows, D)).astype(np.float32))

    y, s, mean, rstd = layer_norm_fwd_raw(_dev_bf16(x, dev), _f32(g, dev), _f32(b, dev), 1e-5,
                                          residual=_dev_bf16(r, dev) if residual else None)
    torch.cuda.synchronize()
    xin = x
    if residual:
        xin = ops.bf16_round(x + r)                       # fp32 add, then RNE to bf16
        assert np.array_equal(_np(s), xin)
    ref, (xh, rs) = om._ln_fwd(xin.astype(np.float64), g.astype(np.float64), b.astype(np.float64), 1e-5)
    assert rel_l2(_np(y), ref) <= 4e-3
    np.testing.assert_allclose(_np(mean), xin.astype(np.float64).mean(-1), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(_np(rstd), rs[:, 0], rtol=1e-5)

    xin_dev = s if residual else _dev_bf16(x, dev)
    outs = [layer_norm_bwd_raw(_dev_bf16(dy, dev), xin_dev, mean, rstd, _f32(g, dev),
                               dres=_dev_bf16(dres, dev) if residual else None) for _ in range(2)]
    torch.cuda.synchronize()
    dx, dg, db = om._ln_bwd(dy.astype(np.float64), g.astype(np.float64), (xh, rs))
    if residual:
        dx = dx + dres
    assert rel_l2(_np(outs[0][0]), dx) <= 1e-2
    assert rel_l2(_np(outs[0][1]), dg) <= 1e-4
    assert rel_l2(_np(outs[0][2]), db) <= 1e-4
    for a, c in zip(outs[0], outs[1]):
        assert torch.equal(a, c)                           # fixed reduction order


def test_layernorm_autograd_chain(dev):
    """add_layer_norm: gradients w.r.t. x and r are equal and include the LN path."""
    import torch
    from nlearn_amd.kernels.fused import add_layer_norm

    rng = np.random.default_rng(3)
    rows, D = 96, 512
    x = _dev_bf16(rng.standard_normal((2, rows // 2, D)), dev).requires_grad_(True)
    r = _dev_bf16(rng.standard_normal((2, rows // 2, D)), dev).requires_grad_(True)
    g = _f32(1 + 0.1 * rng.standard_normal(D), dev).requires_grad_(True)
    b = _f32(0.1 * rng.standard_normal(D), dev).requires_grad_(True)
    wy = _dev_bf16(rng.standard_normal((2, rows // 2, D)), dev)
    ws = _dev_bf16(rng.standard_normal((2, rows // 2, D)), dev)
    y, s = add_layer_norm(x, r, g, b)
    ((y.float() * wy.float()).sum() + (s.float() * ws.float()).sum()).backward()
    torch.cuda.synchronize()
    # float64 reference of the same composition from the saved sum
    xs = torch.tensor(_np(s), dtype=torch.float64, requires_grad=True)
    g64 = torch.tensor(_np(g), dtype=torch.float64, requires_grad=True)
    b64 = torch.tensor(_np(b), dtype=torch.float64, requires_grad=True)
    yr = torch.nn.functional.layer_norm(xs, (D,), g64, b64, 1e-5)
    ((yr * torch.tensor(_np(wy), dtype=torch.float64)).sum()
     + (xs * torch.tensor(_np(ws), dtype=torch.float64)).sum()).backward()
    assert torch.equal(x.grad, r.grad)
    assert rel_l2(_np(x.grad), xs.grad.numpy()) <= 1e-2
    assert rel_l2(_np(g.grad), g64.grad.numpy()) <= 1e-4
    assert rel_l2(_np(b.grad), b64.grad.numpy()) <= 1e-4


# ---------------------------------------------------------------------------
# column sums
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 9), (64, 512), (65, 513), (1000, 2048), (16384, 512),
                                       (300, 50257)])
def test_colsum_exact_integers(dev, rows, cols):
    import torch
    from nlearn_amd.kernels.fused import colsum

    rng = np.random.default_rng(rows + cols)
    x = rng.integers(-8, 9, (rows, cols)).astype(np.float32)
    xd = _dev_bf16(x, dev)
    if cols % 8:  # a padded row stride, as the GEMM outputs have
        ld = (cols + 7) // 8 * 8
        buf = torch.zeros((rows, ld), dtype=torch.bfloat16, device=dev)
        buf[:, :cols] = xd
        xd = buf[:, :cols]
    out = colsum(xd)
    torch.cuda.synchronize()
    assert np.array_equal(_np(out), x.sum(0))


# ---------------------------------------------------------------------------
# GEMM epilogues
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("opB", ["N", "T"])
@pytest.mark.parametrize("M,N,K", [(1, 8, 16), (100, 1001, 70), (300, 520, 256), (512, 2048, 512),
                                   (256, 512, 4096), (4100, 4000, 256)])
def test_gemm_bias_and_gelu_epilogues(dev, M, N, K, opB):
    """Bias, bias+GELU and GELU' epilogues, exact on integer inputs, with B
    stored [K, N] (opB "N") and [N, K] (opB "T"). K = 16 and 70 end in a ragged
    K tail; K = 4096 splits K (epilogue after the reduction); (4100, 4000, 256)
    has enough tiles for the persistent kernel (bias and bias + GELU
    epilogues, ragged edge tiles)."""
    import torch
    from nlearn_amd.kernels.gemm import EPI_BIAS, EPI_BIAS_GELU, EPI_DGELU, gemm_raw, padded_empty

    rng = np.random.default_rng(M + N + K)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    bias = rng.integers(-20, 21, N).astype(np.float32) / 4      # exact quarters
    Ad, biasd = _dev_bf16(A, dev), _f32(bias, dev)
    Bd = _dev_bf16(B if opB == "N" else np.ascontiguousarray(B.T), dev)
    acc = ops.gemm(A, B) + bias                                   # exact (integers / quarters < 2^24)

    c = gemm_raw(Ad, Bd, "N", opB, epi=EPI_BIAS, bias=biasd)                 # fp32 out
    cb = gemm_raw(Ad, Bd, "N", opB, out_dtype=torch.bfloat16, epi=EPI_BIAS, bias=biasd)
    u = padded_empty(M, N, torch.bfloat16, dev)
    h = gemm_raw(Ad, Bd, "N", opB, out=padded_empty(M, N, torch.bfloat16, dev), epi=EPI_BIAS_GELU, bias=biasd,
                 aux=u)
    # backward form: C = (A . B) * gelu'(u) with a scaled product so gelu' varies
    hs = gemm_raw(Ad, Bd, "N", opB, out_dtype=torch.float32, alpha=0.25, epi=EPI_DGELU, aux=u)
    hb = gemm_raw(Ad, Bd, "N", opB, out_dtype=torch.bfloat16, alpha=0.25, epi=EPI_DGELU, aux=u)
    torch.cuda.synchronize()
    assert np.array_equal(_np(c), acc)
    assert np.array_equal(_np(cb), ops.bf16_round(acc))
    u_ref = ops.bf16_round(acc)
    assert np.array_equal(_np(u), u_ref)
    g_ref, t = om._gelu(u_ref.astype(np.float64))
    assert rel_l2(_np(h), g_ref) <= 4e-3
    assert np.abs(_np(h) - g_ref).max() <= np.abs(g_ref).max() * 2 ** -8 + 1e-6
    d_ref = om._gelu_bwd(0.25 * ops.gemm(A, B), u_ref.astype(np.float64), t)
    assert rel_l2(_np(hs), d_ref) <= 1e-5
    # the bf16 output is the fp32 one rounded once
    assert np.array_equal(_np(hb), ops.bf16_round(_np(hs)))


def test_gemm_epilogues_with_split_k(dev):
    """Weight-gradient-like shape (split K): the epilogue runs after the ordered reduction."""
    import torch
    from nlearn_amd.kernels.gemm import EPI_BIAS, EPI_DGELU, gemm_raw, padded_empty
    from nlearn_amd import _lib

    M, N, K = 512, 520, 8192
    assert _lib.load().nl_gemm_ws_bytes(0, 0, M, N, K) > 0        # this shape does split
    rng = np.random.default_rng(11)
    A = rng.integers(-1, 2, (M, K)).astype(np.float32)
    B = rng.integers(-1, 2, (K, N)).astype(np.float32)
    bias = np.arange(N, dtype=np.float32) - 260
    u = ops.bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    Ad, Bd = _dev_bf16(A, dev), _dev_bf16(B, dev)
    c = gemm_raw(Ad, Bd, epi=EPI_BIAS, bias=_f32(bias, dev))
    ud = padded_empty(M, N, torch.bfloat16, dev)
    ud.copy_(_dev_bf16(u, dev))
    d = gemm_raw(Ad, Bd, out_dtype=torch.float32, alpha=1e-3, epi=EPI_DGELU, aux=ud)
    torch.cuda.synchronize()
    assert np.array_equal(_np(c), ops.gemm(A, B) + bias)
    _, t = om._gelu(u.astype(np.float64))
    assert rel_l2(_np(d), om._gelu_bwd(1e-3 * ops.gemm(A, B), u.astype(np.float64), t)) <= 1e-5


def test_ffn_autograd_vs_float64(dev):
    import torch
    from nlearn_amd.kernels.fused import ffn

    rng = np.random.default_rng(5)
    Bt, S, D, F = 2, 64, 128, 512
    x = _dev_bf16(rng.standard_normal((Bt, S, D)), dev).requires_grad_(True)
    W1 = _f32(rng.standard_normal((D, F)) * 0.05, dev).requires_grad_(True)
    b1 = _f32(rng.standard_normal(F) * 0.1, dev).requires_grad_(True)
    W2 = _f32(rng.standard_normal((F, D)) * 0.05, dev).requires_grad_(True)
    b2 = _f32(rng.standard_normal(D) * 0.1, dev).requires_grad_(True)
    dy = _dev_bf16(rng.standard_normal((Bt, S, D)), dev)
    y = ffn(x, W1, b1, W2, b2)
    y.backward(dy)
    torch.cuda.synchronize()

    def t64(a):
        return torch.tensor(_np(a), dtype=torch.float64, requires_grad=True)

    xr, b1r, b2r = t64(x), t64(b1), t64(b2)
    W1r = torch.tensor(ops.bf16_round(_np(W1)), dtype=torch.float64, requires_grad=True)
    W2r = torch.tensor(ops.bf16_round(_np(W2)), dtype=torch.float64, requires_grad=True)
    yr = torch.nn.functional.gelu(xr @ W1r + b1r, approximate="tanh") @ W2r + b2r
    yr.backward(torch.tensor(_np(dy), dtype=torch.float64))
    assert rel_l2(_np(y), yr.detach().numpy()) <= 1e-2
    assert x.grad.dtype == torch.bfloat16
    for got, want in [(x.grad, xr.grad), (W1.grad, W1r.grad), (b1.grad, b1r.grad), (W2.grad, W2r.grad),
                      (b2.grad, b2r.grad)]:
        assert rel_l2(_np(got), want.numpy()) <= 2e-2
    assert all(p.grad.dtype == torch.float32 for p in (W1, b1, W2, b2))


# ---------------------------------------------------------------------------
# embedding
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("B,S,V,D,P", [(1, 1, 7, 4, 1), (3, 37, 1000, 64, 40), (32, 512, 50257, 512, 512)])
def test_embedding_fwd_bwd(dev, B, S, V, D, P):
    import torch
    from nlearn_amd.kernels.fused import embedding

    rng = np.random.default_rng(B * S + V)
    ids = rng.integers(0, V, (B, S)).astype(np.int32)
    ids[0, 0] = V - 1
    tok = rng.standard_normal((V, D)).astype(np.float32) * 0.02
    pos = rng.standard_normal((P, D)).astype(np.float32) * 0.02
    tokd = _f32(tok, dev).requires_grad_(True)
    posd = _f32(pos, dev).requires_grad_(True)
    out = embedding(torch.from_numpy(ids).to(dev), tokd, posd)
    dx = rng.integers(-4, 5, (B, S, D)).astype(np.float32)
    out.backward(_dev_bf16(dx, dev))
    torch.cuda.synchronize()
    assert np.array_equal(_np(out), ops.bf16_round(tok[ids] + pos[:S][None]))
    dtok = np.zeros((V, D))
    np.add.at(dtok, ids.reshape(-1), dx.reshape(-1, D))
    assert np.array_equal(_np(tokd.grad), dtok)                   # small integers: any order is exact
    dpos = np.zeros((P, D), np.float32)
    dpos[:S] = dx.sum(0)
    assert np.array_equal(_np(posd.grad), dpos)


@pytest.mark.parametrize("pattern", ["skewed", "one_id", "all_outside"])
def test_embedding_bwd_sums_in_token_order(dev, pattern):
    """Skewed ids (one id on a quarter of the tokens, a few hot ones, runs of
    the same id) and non-integer gradients, where the summation order shows in
    the last bits: the token table's gradient is np.add.at's float32 sum, in
    increasing token order, bit for bit; rows no token uses come back zero in
    a table that started as NaN; ids outside [0, vocab) add nothing. Also
    every token on one id (one bucket's lists take the whole one-entry-per-
    token workspace) and every id outside the table (empty lists)."""
    import torch
    from nlearn_amd import _lib

    B, S, V, D = 8, 1000, 3000, 512
    rng = np.random.default_rng(11)
    ids = rng.integers(0, V, (B, S)).astype(np.int32)
    ids[rng.random((B, S)) < 0.25] = 17
    ids[:, 100:140] = 2999
    ids[3, 7] = V
    ids[5, 9] = -4
    if pattern == "one_id":
        ids[:] = 1234
    elif pattern == "all_outside":
        ids[:] = V + rng.integers(0, 5, (B, S)).astype(np.int32)
    dx = ops.bf16_round(rng.standard_normal((B, S, D)).astype(np.float32))
    dtok = torch.full((V, D), float("nan"), device=dev)
    dpos = torch.zeros((S, D), device=dev)
    outs = []
    wsb = int(_lib.load().nl_embedding_bwd_ws_bytes(B, S, D, V))
    ws = torch.empty(wsb // 4, dtype=torch.int32, device=dev)
    for _ in range(2):
        ws.fill_(-1)                                              # stale workspace contents must not matter
        _lib.call("nl_embedding_bwd", torch.cuda.current_stream().cuda_stream, B, S, D, V,
                  torch.from_numpy(ids).to(dev).data_ptr(), _dev_bf16(dx, dev).data_ptr(), dtok.data_ptr(),
                  dpos.data_ptr(), 0, ws.data_ptr(), wsb)
        torch.cuda.synchronize()
        outs.append(_np(dtok).copy())
    flat, rows = ids.reshape(-1), dx.reshape(-1, D)
    keep = (flat >= 0) & (flat < V)
    ref = np.zeros((V, D), np.float32)
    np.add.at(ref, flat[keep], rows[keep])
    assert np.array_equal(outs[0], ref)
    assert np.array_equal(outs[1], outs[0])
    ref_pos = np.zeros((S, D), np.float32)
    for b in range(B):                                            # batch order, as the kernel
        ref_pos += dx[b]
    assert np.array_equal(_np(dpos), ref_pos)


def test_embedding_invalid_ids_give_nan_rows(dev):
    import torch
    from nlearn_amd.kernels.fused import embedding

    tok = torch.ones((10, 8), device=dev)
    pos = torch.zeros((4, 8), device=dev)
    ids = torch.tensor([[1, 10, -1, 9]], dtype=torch.int32, device=dev)
    out = embedding(ids, tok, pos).float().cpu()
    assert torch.isnan(out[0, 1]).all() and torch.isnan(out[0, 2]).all()
    assert (out[0, 0] == 1).all() and (out[0, 3] == 1).all()


@pytest.mark.parametrize("B,S,P", [(2, 64, 64), (3, 37, 40)])
def test_embedding_layer_norm_matches_the_composition(dev, B, S, P):
    """embedding_layer_norm == layer_norm(embedding(.)) with both outputs' gradients, its
    parameter gradients written into main_grad buffers that start as NaN (every element
    must be overwritten; the position table past S must come back zero)."""
    import torch
    from nlearn_amd.kernels.fused import embedding, embedding_layer_norm, layer_norm

    V, D = 1000, 64
    rng = np.random.default_rng(B + S + P)
    ids = torch.from_numpy(rng.integers(0, V, (B, S)).astype(np.int32)).to(dev)
    tables = [rng.standard_normal((V, D)) * 0.5, rng.standard_normal((P, D)) * 0.5,
              1 + 0.1 * rng.standard_normal(D), 0.1 * rng.standard_normal(D)]
    dy = _dev_bf16(rng.standard_normal((B, S, D)), dev)
    dx = _dev_bf16(rng.standard_normal((B, S, D)), dev)
    ref = [_f32(a, dev).requires_grad_(True) for a in tables]
    x = embedding(ids, ref[0], ref[1])
    h = layer_norm(x, ref[2], ref[3])
    torch.autograd.backward([h, x], [dy, dx])
    fused = [_f32(a, dev).requires_grad_(True) for a in tables]
    for t in fused:
        t.main_grad = torch.full_like(t, float("nan"))
    h1, x1 = embedding_layer_norm(ids, *fused)
    torch.autograd.backward([h1, x1], [dy, dx])
    torch.cuda.synchronize()
    assert torch.equal(h1, h) and torch.equal(x1, x)
    for got, want in zip(fused, ref):
        assert got.grad is None
        g = _np(got.main_grad)
        assert np.isfinite(g).all()
        # the fused backward adds x's gradient in fp32 before one bf16 rounding,
        # the composition rounds the LayerNorm's dx to bf16 first
        assert rel_l2(g, _np(want.grad)) <= 1e-2
    assert not _np(fused[1].main_grad)[S:].any()


@pytest.mark.parametrize("shapes", [[(16384, 512), (16384, 512), (300, 512)], [(257, 512), (33, 1024), (5, 4096)]])
def test_layernorm_deferred_param_sums_match_bitwise(dev, shapes):
    """A chain of nl_layernorm_bwd_deferred calls (each launch reducing the previous call's
    partials) closed by nl_layernorm_param_sums gives the dx, dgamma and dbeta of separate
    nl_layernorm_bwd calls bit for bit, including an accumulating reduction."""
    import torch
    from nlearn_amd import _lib
    from nlearn_amd.kernels import fused

    rng = np.random.default_rng(len(shapes) + shapes[-1][0])
    st = torch.cuda.current_stream(dev).cuda_stream
    calls = []
    for rows, D in shapes:
        x = _dev_bf16(rng.standard_normal((rows, D)), dev)
        dy = _dev_bf16(rng.standard_normal((rows, D)), dev)
        g = _f32(1 + 0.1 * rng.standard_normal(D), dev)
        b = _f32(0.1 * rng.standard_normal(D), dev)
        _, _, mean, rstd = fused.layer_norm_fwd_raw(x, g, b, 1e-5)
        calls.append((rows, D, x, dy, g, mean, rstd, _f32(rng.standard_normal(D), dev), _f32(rng.standard_normal(D), dev)))
    accumulate = [0, 1, 0]
    plain, chained, keep, pending = [], [], [], None
    for (rows, D, x, dy, g, mean, rstd, g0, b0), acc in zip(calls, accumulate):
        wsb = int(_lib.load().nl_layernorm_bwd_ws_bytes(rows, D))
        outs = []
        for deferred in (False, True):
            dx = torch.empty_like(x)
            dg, db = g0.clone(), b0.clone()
            ws = torch.empty(wsb // 4, dtype=torch.float32, device=dev)
            if not deferred:
                _lib.call("nl_layernorm_bwd", st, rows, D, dy.data_ptr(), x.data_ptr(), mean.data_ptr(),
                          rstd.data_ptr(), g.data_ptr(), None, dx.data_ptr(), dg.data_ptr(), db.data_ptr(), acc,
                          ws.data_ptr(), wsb)
            else:
                prev = (pending[0], pending[1], pending[2].data_ptr(), pending[3].data_ptr(), pending[4].data_ptr(),
                        pending[5]) if pending else (0, 0, None, None, None, 0)
                _lib.call("nl_layernorm_bwd_deferred", st, rows, D, dy.data_ptr(), x.data_ptr(), mean.data_ptr(),
                          rstd.data_ptr(), g.data_ptr(), None, dx.data_ptr(), ws.data_ptr(), wsb, *prev)
                keep.append(ws)      # partials stay alive until a later launch has reduced them
                pending = (rows, D, ws, dg, db, acc)
            outs.append((dx, dg, db))
        plain.append(outs[0])
        chained.append(outs[1])
    rows, D, ws, dg, db, acc = pending
    _lib.call("nl_layernorm_param_sums", st, rows, D, ws.data_ptr(), dg.data_ptr(), db.data_ptr(), acc)
    torch.cuda.synchronize()
    assert len(chained) == len(plain) == len(shapes)
    for (dx0, dg0, db0), (dx1, dg1, db1) in zip(plain, chained):
        assert torch.equal(dx0.view(torch.int16), dx1.view(torch.int16))
        assert torch.equal(dg0, dg1) and torch.equal(db0, db1)
