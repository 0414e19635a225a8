"""CPU pins of the op-level oracle (oracle/ops.py) against independent
implementations and closed forms. Each check is chosen so that a plausible
mistake (a dropped term, a wrong sign or index, a transposed operand) fails."""
import math

import numpy as np
import pytest
import torch

from oracle import ops


def test_bf16_rounding_matches_torch_bit_for_bit():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1e-40, -1e-40, 3.3895e38, -3.3895e38, np.inf, -np.inf], np.float32),
                        # exact ties: RNE must pick the even neighbour
                        (np.arange(1, 1000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ops.bf16_bits(x), ref)
    nan = ops.bf16_to_f32(ops.bf16_bits(np.array([np.nan], np.float32)))
    assert np.isnan(nan[0])


@pytest.mark.parametrize("opA,opB", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
def test_gemm_transposes_and_exact_integers(opA, opB):
    rng = np.random.default_rng(1)
    A = rng.integers(-4, 5, (37, 53)).astype(np.float32)
    B = rng.integers(-4, 5, (53, 29)).astype(np.float32)
    ref = A.astype(np.int64) @ B.astype(np.int64)     # exact integer product
    As = A.T.copy() if opA == "T" else A
    Bs = B.T.copy() if opB == "T" else B
    assert np.array_equal(ops.gemm(As, Bs, opA, opB), ref)


def _torch_attention(q, k, v, causal):
    s = q @ k.transpose(-1, -2) / math.sqrt(q.shape[-1])
    if causal:
        S = q.shape[1]
        s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    return torch.softmax(s, -1) @ v, torch.logsumexp(s, -1)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("n,s,d", [(2, 16, 8), (3, 37, 64)])
def test_flash_forward_backward_vs_float64_autograd(n, s, d, causal):
    rng = np.random.default_rng(n * s + d)
    Q, K, V, dO = (rng.standard_normal((n, s, d)) for _ in range(4))
    O, L = ops.flash_fwd(Q, K, V, causal=causal)
    dQ, dK, dV, D = ops.flash_bwd(Q, K, V, dO, causal=causal)
    tq, tk, tv = (torch.from_numpy(a).requires_grad_(True) for a in (Q, K, V))
    tO, tL = _torch_attention(tq, tk, tv, causal)
    tO.backward(torch.from_numpy(dO))
    np.testing.assert_allclose(O, tO.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(L, tL.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dQ, tq.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dK, tk.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dV, tv.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(D, (dO * O).sum(-1), rtol=1e-12)


def test_flash_closed_forms_and_invariants():
    rng = np.random.default_rng(5)
    n, s, d = 2, 24, 16
    Q, K, V, dO = (rng.standard_normal((n, s, d)) for _ in range(4))
    O, L = ops.flash_fwd(Q, K, V)
    # the first query sees only the first key
    np.testing.assert_allclose(O[:, 0], V[:, 0], rtol=1e-12)
    np.testing.assert_allclose(L[:, 0], (Q[:, 0] * K[:, 0]).sum(-1) / math.sqrt(d), rtol=1e-12)
    # identical keys -> uniform weights over the causal prefix -> prefix mean of V
    Ke = np.repeat(K[:, :1], s, axis=1)
    Oe, _ = ops.flash_fwd(Q, Ke, V)
    prefix_mean = np.cumsum(V, 1) / np.arange(1, s + 1)[None, :, None]
    np.testing.assert_allclose(Oe, prefix_mean, rtol=1e-10, atol=1e-12)
    dQ, dK, dV, _ = ops.flash_bwd(Q, K, V, dO)
    np.testing.assert_allclose(dV.sum(1), dO.sum(1), rtol=1e-10)      # rows of P sum to 1
    np.testing.assert_allclose(dK.sum(1), 0.0, atol=1e-10)            # softmax shift invariance
    # finite differences on one entry of K
    eps = 1e-6
    K2 = K.copy()
    K2[1, 3, 5] += eps
    O2, _ = ops.flash_fwd(Q, K2, V)
    fd = ((O2 - O) * dO).sum() / eps
    assert fd == pytest.approx(dK[1, 3, 5], rel=1e-4, abs=1e-7)


def test_flash_never_uses_future_keys():
    rng = np.random.default_rng(6)
    Q, K, V = (rng.standard_normal((1, 10, 8)) for _ in range(3))
    K2, V2 = K.copy(), V.copy()
    K2[:, 6:] = 1e6
    V2[:, 6:] = -1e6
    O1, L1 = ops.flash_fwd(Q, K, V)
    O2, L2 = ops.flash_fwd(Q, K2, V2)
    np.testing.assert_allclose(O1[:, :6], O2[:, :6], rtol=1e-12)
    np.testing.assert_allclose(L1[:, :6], L2[:, :6], rtol=1e-12)


def test_ce_vs_torch_and_invariants():
    rng = np.random.default_rng(7)
    M, V = 33, 101
    x = rng.standard_normal((M, V)) * 3
    t = rng.integers(0, V, M)
    loss, lse, dl = ops.ce(x, t)
    tx = torch.from_numpy(x).requires_grad_(True)
    tl = torch.nn.functional.cross_entropy(tx, torch.from_numpy(t))
    tl.backward()
    assert loss.mean() == pytest.approx(tl.item(), rel=1e-12)
    np.testing.assert_allclose(dl, tx.grad.numpy(), rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(lse, torch.logsumexp(torch.from_numpy(x), -1).numpy(), rtol=1e-12)
    np.testing.assert_allclose(dl.sum(1), 0.0, atol=1e-14)
    assert (dl[np.arange(M), t] < 0).all() and (np.delete(dl.ravel(), np.arange(M) * V + t) > 0).all()
    assert (loss >= 0).all()
    # uniform logits give exactly ln V
    l0, _, _ = ops.ce(np.zeros((4, V)), np.arange(4))
    np.testing.assert_allclose(l0, math.log(V), rtol=1e-14)


def test_linear_ce_oracle_pins():
    """ops.linear_ce (the chunked restatement of linear_cross_entropy) against
    checks that do not share its code: torch float64 autograd of
    CE(X @ W) for the loss and both gradients (unrounded), chunk-size
    independence (a wrong online rescale would break it), and W = 0, where the
    loss is exactly ln V and dW = X^T (1/V - onehot) / M."""
    rng = np.random.default_rng(11)
    M, D, V = 13, 7, 50
    X = rng.standard_normal((M, D))
    W = rng.standard_normal((D, V)) * 0.7
    t = rng.integers(0, V, M)
    loss, lse, dX, dW = ops.linear_ce(X, W, t, chunk=8, round_bf16=False)
    tX = torch.from_numpy(X).requires_grad_(True)
    tW = torch.from_numpy(W).requires_grad_(True)
    tl = torch.nn.functional.cross_entropy(tX @ tW, torch.from_numpy(t))
    tl.backward()
    assert loss == pytest.approx(tl.item(), rel=1e-12)
    np.testing.assert_allclose(dX, tX.grad.numpy(), rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(dW, tW.grad.numpy(), rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(lse, torch.logsumexp(tX.detach() @ tW.detach(), -1).numpy(), rtol=1e-12)
    for ch in (1, 7, 49, 50, 4096):
        l2, lse2, dX2, dW2 = ops.linear_ce(X, W, t, chunk=ch, round_bf16=False)
        assert l2 == pytest.approx(loss, rel=1e-12)
        np.testing.assert_allclose(dX2, dX, rtol=1e-10, atol=1e-14)
        np.testing.assert_allclose(dW2, dW, rtol=1e-10, atol=1e-14)
    l0, lse0, dX0, dW0 = ops.linear_ce(X, np.zeros((D, V)), t, chunk=16)
    assert l0 == pytest.approx(math.log(V), rel=1e-14)
    np.testing.assert_allclose(dX0, 0.0, atol=0)
    oh = np.zeros((M, V))
    oh[np.arange(M), t] = 1.0
    np.testing.assert_allclose(dW0, X.T @ ops.bf16_round((1.0 / V - oh) / M).astype(np.float64), rtol=1e-12)
    # the rounded form equals the unfused composition CE(bf16(X @ W)) with bf16 dlogits
    Xb, Wb = ops.bf16_round(X).astype(np.float64), ops.bf16_round(W).astype(np.float64)
    lr, lser, dXr, dWr = ops.linear_ce(Xb, Wb, t, chunk=16)
    cl, clse, cdl = ops.ce(ops.bf16_round(Xb @ Wb), t)
    assert lr == pytest.approx(cl.mean(), rel=1e-12)
    np.testing.assert_allclose(lser, clse, rtol=1e-12)
    np.testing.assert_allclose(dWr, Xb.T @ ops.bf16_round(cdl).astype(np.float64), rtol=1e-10, atol=1e-14)


def test_gelu_and_layernorm_pieces_vs_torch_float64():
    """The elementwise pieces of the model oracle against torch's own float64
    implementations (an independent code path): tanh-GELU and its derivative,
    LayerNorm forward and backward (dx, dgamma, dbeta)."""
    from oracle import model_np as om

    rng = np.random.default_rng(8)
    u = rng.standard_normal(4001) * 4
    u[:3] = [0.0, -30.0, 30.0]
    gu, t = om._gelu(u)
    tu = torch.from_numpy(u).requires_grad_(True)
    ref = torch.nn.functional.gelu(tu, approximate="tanh")
    np.testing.assert_allclose(gu, ref.detach().numpy(), rtol=1e-12, atol=1e-15)
    ref.backward(torch.ones_like(ref))
    np.testing.assert_allclose(om._gelu_bwd(np.ones_like(u), u, t), tu.grad.numpy(), rtol=1e-10, atol=1e-14)
    # closed forms: gelu(0) = 0, gelu'(0) = 1/2, saturation at +-30
    assert gu[0] == 0.0 and gu[1] == pytest.approx(0.0, abs=1e-12) and gu[2] == pytest.approx(30.0)

    x = rng.standard_normal((37, 48)) * 3 + 1
    g = rng.standard_normal(48)
    b = rng.standard_normal(48)
    dy = rng.standard_normal((37, 48))
    y, cache = om._ln_fwd(x, g, b, 1e-5)
    tx = torch.from_numpy(x).requires_grad_(True)
    tg = torch.from_numpy(g).requires_grad_(True)
    tb = torch.from_numpy(b).requires_grad_(True)
    ty = torch.nn.functional.layer_norm(tx, (48,), tg, tb, 1e-5)
    np.testing.assert_allclose(y, ty.detach().numpy(), rtol=1e-10, atol=1e-12)
    ty.backward(torch.from_numpy(dy))
    dx, dg, db = om._ln_bwd(dy, g, cache)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(dg, tg.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(db, tb.grad.numpy(), rtol=1e-12, atol=1e-12)
    # invariants: dx is orthogonal to the all-ones vector; with eps = 0 also to xh
    np.testing.assert_allclose(dx.sum(-1), 0.0, atol=1e-10)
    _, c0 = om._ln_fwd(x, g, b, 0.0)
    dx0, _, _ = om._ln_bwd(dy, g, c0)
    np.testing.assert_allclose((dx0 * c0[0]).sum(-1), 0.0, atol=1e-10)
