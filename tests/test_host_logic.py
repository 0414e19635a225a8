"""CPU checks of host-side logic that needs no GPU."""
import pytest


def test_kernel_ready_copies_overlapping_rows():
    """A broadcast view (row stride 0) must not reach a kernel as a matrix
    with ld = #columns: _kernel_ready copies it, and _ld refuses it."""
    import torch
    from nlearn_amd.kernels.gemm import _kernel_ready, _ld

    b = torch.ones(8, dtype=torch.bfloat16).expand(4, 8)
    assert b.stride() == (0, 1)
    with pytest.raises(ValueError, match="overlap"):
        _ld(b)
    r = _kernel_ready(b)
    assert r.shape == (4, 8) and r.stride(0) >= 8 and torch.equal(r, b)
    # a dense or padded matrix is passed through untouched
    d = torch.zeros((4, 16), dtype=torch.bfloat16)[:, :12]
    assert _kernel_ready(d).data_ptr() == d.data_ptr() and _ld(d) == 16
    one = torch.zeros((1, 12), dtype=torch.bfloat16)
    assert _ld(one) == 16
