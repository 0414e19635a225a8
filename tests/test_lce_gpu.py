"""GPU parity of the fused LM head + cross-entropy (linear_cross_entropy,
cross_entropy.py:84-170) through the C ABI (nl_lce_fwd, nl_lce_bwd_dlogits).

* Against the float64 oracle (ops.linear_ce with bf16-rounded logits and
  dlogits, the reference's chunked algorithm) at the reference's own check
  shapes (check_lce.py: (256, 64, 2050), (512, 256, 12000)) and ragged ones:
  loss abs <= 1e-3, lse rel 1e-5, dX / dW rel-L2 <= 1e-2.
* Against the unfused path (linear -> cross_entropy) at the BASELINE size
  (16384, 512, 50257): the same bf16 logits feed both, so the loss agrees to
  1e-5 and the gradients to rel-L2 1e-3.
* The sliced backward (NLEARN_LCE_CHUNK) equals the one-pass backward.
* A target outside [0, V) gives a NaN loss for its row only.
"""
import numpy as np
import pytest

from conftest import rel_l2
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


def _weight(W, dev):
    from nlearn_amd.model import device_param

    return device_param(np.asarray(W, np.float32), dev)   # fp32 leaf, padded row stride like the model's


@pytest.mark.parametrize("M,D,V", [(256, 64, 2050), (512, 256, 12000), (33, 64, 257), (300, 128, 5000)])
def test_lce_vs_oracle(dev, M, D, V):
    import torch
    from nlearn_amd.kernels.cross_entropy import linear_cross_entropy

    rng = np.random.default_rng(M + D + V)
    X = ops.bf16_round(rng.standard_normal((M, D)) * 0.1)
    W = ops.bf16_round(rng.standard_normal((D, V)) * 0.5)
    t = rng.integers(0, V, M)
    Xd = _dev_bf16(X, dev).requires_grad_(True)
    Wd = _weight(W, dev)
    loss = linear_cross_entropy(Xd, Wd, torch.from_numpy(t).to(dev))
    loss.backward()
    torch.cuda.synchronize()
    lr, lser, dXr, dWr = ops.linear_ce(X, W, t, chunk=4096)
    assert abs(loss.item() - lr) <= 1e-3
    assert rel_l2(_np(Xd.grad), dXr) <= 1e-2
    assert rel_l2(_np(Wd.grad), dWr) <= 1e-2


def test_lce_fwd_rows_and_invalid_target(dev):
    """Per-row loss and lse from nl_lce_fwd; an out-of-range target poisons only its row."""
    import torch
    from nlearn_amd import _lib

    rng = np.random.default_rng(5)
    M, D, V = 300, 64, 3001
    X = ops.bf16_round(rng.standard_normal((M, D)) * 0.2)
    W = ops.bf16_round(rng.standard_normal((D, V)))
    t = rng.integers(0, V, M).astype(np.int32)
    t[7], t[100] = V, -1
    Xd = _dev_bf16(X, dev)
    Wd = torch.zeros((D, (V + 7) // 8 * 8), dtype=torch.bfloat16, device=dev)
    Wd[:, :V] = _dev_bf16(W, dev)
    td = torch.from_numpy(t).to(dev)
    loss = torch.empty(M, dtype=torch.float32, device=dev)
    lse = torch.empty(M, dtype=torch.float32, device=dev)
    wsb = int(_lib.load().nl_lce_ws_bytes(M, V))
    ws = torch.empty(wsb // 4 + 4, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    _lib.call("nl_lce_fwd", st, M, D, V, Xd.data_ptr(), D, Wd.data_ptr(), Wd.shape[1], td.data_ptr(),
              loss.data_ptr(), lse.data_ptr(), ws.data_ptr(), wsb)
    torch.cuda.synchronize()
    logits = ops.bf16_round(X.astype(np.float64) @ W.astype(np.float64)).astype(np.float64)
    ok = np.ones(M, bool)
    ok[[7, 100]] = False
    cl, clse, _ = ops.ce(logits[ok], t[ok])
    got = _np(loss)
    assert np.isnan(got[[7, 100]]).all()
    np.testing.assert_allclose(got[ok], cl, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(_np(lse)[ok], clse, rtol=1e-5)
    np.testing.assert_allclose(_np(lse)[~ok], ops.ce(logits[~ok], np.zeros(2, np.int64))[1], rtol=1e-5)
    with pytest.raises(_lib.NlError):   # workspace too small: refused before any launch
        _lib.call("nl_lce_fwd", st, M, D, V, Xd.data_ptr(), D, Wd.data_ptr(), Wd.shape[1], td.data_ptr(),
                  loss.data_ptr(), lse.data_ptr(), ws.data_ptr(), wsb - 16)


def test_lce_matches_unfused_path_at_baseline_size(dev):
    import torch
    from nlearn_amd.kernels.cross_entropy import cross_entropy, linear_cross_entropy
    from nlearn_amd.kernels.gemm import linear

    M, D, V = 16384, 512, 50257
    g = torch.Generator(device=dev).manual_seed(3)
    X = (torch.randn((M, D), generator=g, device=dev) * 0.5).to(torch.bfloat16)
    W = _weight(np.random.default_rng(3).standard_normal((D, V)).astype(np.float32) * 0.05, dev)
    t = torch.randint(0, V, (M,), generator=g, device=dev)
    Xa = X.clone().requires_grad_(True)
    la = cross_entropy(linear(Xa, W), t, inplace=True)
    la.backward()
    dWa = W.grad.clone()
    W.grad = None
    Xb = X.clone().requires_grad_(True)
    lb = linear_cross_entropy(Xb, W, t)
    lb.backward()
    torch.cuda.synchronize()
    assert abs(la.item() - lb.item()) <= 1e-5
    assert rel_l2(_np(Xb.grad), _np(Xa.grad)) <= 1e-3
    assert rel_l2(_np(W.grad), _np(dWa)) <= 1e-3


def test_lce_sliced_backward_matches_one_pass(dev, monkeypatch):
    import torch
    from nlearn_amd.kernels import cross_entropy as ce

    rng = np.random.default_rng(9)
    M, D, V = 1000, 128, 9001
    X = ops.bf16_round(rng.standard_normal((M, D)) * 0.3)
    W = rng.standard_normal((D, V)).astype(np.float32) * 0.1
    t = torch.from_numpy(rng.integers(0, V, M)).to(dev)
    grads = {}
    for chunk in (0, 2048):
        monkeypatch.setattr(ce, "_LCE_CHUNK", chunk)
        Xd = _dev_bf16(X, dev).requires_grad_(True)
        Wd = _weight(W, dev)
        loss = ce.linear_cross_entropy(Xd, Wd, t)
        loss.backward()
        torch.cuda.synchronize()
        grads[chunk] = (loss.item(), _np(Xd.grad), _np(Wd.grad))
    assert grads[0][0] == grads[2048][0]
    assert rel_l2(grads[2048][1], grads[0][1]) <= 1e-2        # dX: fp32 slice sums vs one bf16 product
    assert rel_l2(grads[2048][2], grads[0][2]) <= 1e-5        # dW: the same columns, other split plans
