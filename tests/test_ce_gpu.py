"""GPU parity of the fused cross-entropy against the float64 oracle.

Tolerances (north_star): loss absolute <= 1e-3, dlogits relative L2 <= 1e-2.
"""
import math

import numpy as np
import pytest

from conftest import GOLDEN, rel_l2
from oracle import ops

pytestmark = pytest.mark.gpu


def _to_dev_bf16(bits, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)


def _np(t):
    import torch

    if t.dtype == torch.bfloat16:
        return ops.bf16_to_f32(t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))
    return t.cpu().numpy()


def test_ce_golden_512x1024(dev):
    import torch
    from nlearn_amd.kernels import cross_entropy as ce

    g = np.load(GOLDEN / "ce_512x1024.npz")
    x = _to_dev_bf16(g["logits"], dev)
    t = torch.from_numpy(g["targets"]).to(dev)
    loss, lse, d = ce.ce_fwd_bwd_raw(x, t)
    torch.cuda.synchronize()
    assert np.abs(_np(loss) - g["loss"]).max() <= 1e-3
    assert np.abs(_np(lse) - g["lse"]).max() <= 1e-3
    assert rel_l2(_np(d)[:64], g["dlogits_head"]) <= 1e-2
    # separate reference-style passes agree with the fused pass
    loss2, lse2 = ce._ce_fwd_raw(x, t)
    d2 = ce._ce_bwd_raw(x, t, lse2)
    torch.cuda.synchronize()
    assert np.abs(_np(loss2) - g["loss"]).max() <= 1e-3
    assert rel_l2(_np(d2)[:64], g["dlogits_head"]) <= 1e-2
    assert np.array_equal(_np(d2), _np(d))


@pytest.mark.parametrize("M,V,ld,inplace", [
    (1, 1, 1, False), (3, 7, 7, False), (5, 9, 16, True), (37, 1000, 1000, False),
    (64, 4097, 4104, True), (19, 50257, 50257, False), (23, 50257, 50264, True),
    (4, 60001, 60001, False),   # beyond the register capacity: generic two-read path
])
def test_ce_ragged_shapes(dev, M, V, ld, inplace):
    import torch
    from nlearn_amd.kernels import cross_entropy as ce

    rng = np.random.default_rng(M * 1000 + V)
    x = (rng.standard_normal((M, V)) * 2.0).astype(np.float32)
    t = rng.integers(0, V, (M,)).astype(np.int32)
    xb = ops.bf16_bits(x)
    buf = torch.zeros((M, ld), dtype=torch.bfloat16, device=dev)
    view = buf[:, :V]
    view.copy_(_to_dev_bf16(xb, dev))
    ref_loss, ref_lse, ref_d = ops.ce(ops.bf16_to_f32(xb), t)
    loss, lse, d = ce.ce_fwd_bwd_raw(view, torch.from_numpy(t).to(dev), inplace=inplace)
    torch.cuda.synchronize()
    assert np.abs(_np(loss) - ref_loss).max() <= 1e-3
    assert np.abs(_np(lse) - ref_lse).max() <= 1e-3
    assert rel_l2(_np(d), ref_d) <= 1e-2
    if inplace:
        assert d.data_ptr() == view.data_ptr()
    if ld > V:  # padding columns untouched
        assert torch.count_nonzero(buf[:, V:]).item() == 0


def test_ce_invalid_target_gives_nan_row(dev):
    import torch
    from nlearn_amd.kernels import cross_entropy as ce

    x = torch.randn(4, 100, device=dev).to(torch.bfloat16)
    t = torch.tensor([0, 100, -1, 5], dtype=torch.int32, device=dev)
    loss, lse, d = ce.ce_fwd_bwd_raw(x, t)
    l = loss.cpu().numpy()
    assert np.isfinite(l[[0, 3]]).all() and np.isnan(l[[1, 2]]).all()
    assert torch.isfinite(d.float()).all()


def test_ce_autograd_and_cotangent(dev):
    import torch
    from nlearn_amd.kernels.cross_entropy import cross_entropy

    rng = np.random.default_rng(3)
    M, V = 96, 3000
    xb = ops.bf16_bits(rng.standard_normal((M, V)).astype(np.float32))
    t = rng.integers(0, V, (M,)).astype(np.int32)
    x = _to_dev_bf16(xb, dev).requires_grad_(True)
    loss = cross_entropy(x.view(8, 12, V), torch.from_numpy(t).to(dev).view(8, 12))
    (loss * 3.0).backward()
    ref_loss, _, ref_d = ops.ce(ops.bf16_to_f32(xb), t)
    assert abs(loss.item() - ref_loss.mean()) <= 1e-3
    assert rel_l2(_np(x.grad), 3.0 * ref_d) <= 1e-2


def test_ce_full_size_properties(dev):
    """(16384, 50257) bf16 ~ N(0, 2): sampled rows vs the oracle, plus
    size-independent properties over every row."""
    import torch
    from nlearn_amd.kernels import cross_entropy as ce

    M, V = 16384, 50257
    gen = torch.Generator(device=dev).manual_seed(1234)
    x = (torch.randn((M, V), generator=gen, device=dev) * 2.0).to(torch.bfloat16)
    t = torch.randint(0, V, (M,), generator=gen, device=dev, dtype=torch.int32)
    rows = np.random.default_rng(0).choice(M, 64, replace=False)
    xs = _np(x[rows]).astype(np.float64)
    loss, lse, d = ce.ce_fwd_bwd_raw(x, t, inplace=True)   # dlogits over the logits
    torch.cuda.synchronize()
    ref_loss, ref_lse, ref_d = ops.ce(xs, t.cpu().numpy()[rows], scale=1.0 / M)
    assert np.abs(_np(loss)[rows] - ref_loss).max() <= 1e-3
    assert rel_l2(_np(d[rows]), ref_d) <= 1e-2
    # every row: sum_v dlogits = 0 (bf16 rounding tolerance), target entry negative
    rs = d.float().sum(1) * M
    assert rs.abs().max().item() < 5e-2
    dt = d.gather(1, t.long().view(-1, 1)).float()
    assert (dt < 0).all()
    mean_loss = ce.mean(loss).item()
    # E[loss] for N(0, s^2) logits ~= ln V + s^2/2
    assert abs(mean_loss - (math.log(V) + 2.0)) < 0.05


@pytest.mark.parametrize("rows,cols,ld,offset", [(300, 50257, 50304, 0), (7, 13, 16, 0), (9, 40, 48, 1)])
def test_scale_by_device_scalar(dev, rows, cols, ld, offset):
    """dlogits *= g (the CE backward's cotangent) in place: bf16(x * g) with one
    RNE rounding per element, on 16-byte aligned rows (8 elements per load,
    ragged tails) and on rows that start off that alignment (element path);
    g == 1 leaves every bit, the padding included, untouched."""
    import torch
    from nlearn_amd.kernels.cross_entropy import scale_by_device_scalar_

    gen = torch.Generator(device="cpu").manual_seed(rows + cols)
    base = torch.randn(rows * ld + offset, generator=gen).to(torch.bfloat16).to(dev)
    x = base[offset:].view(rows, ld)[:, :cols]
    for g in (3.0, 1.0, -0.37):
        before = base.clone()
        scale_by_device_scalar_(x, torch.tensor(g, device=dev))
        torch.cuda.synchronize()
        want = before[offset:].view(rows, ld).clone()
        want[:, :cols] = (want[:, :cols].float() * g).to(torch.bfloat16)
        assert torch.equal(base[offset:].view(rows, ld), want)
        assert torch.equal(base[:offset], before[:offset])
