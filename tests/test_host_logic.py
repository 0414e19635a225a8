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


def test_padded_empty_row_strides():
    """Rows start on 16-byte boundaries; rows of 1024 columns or more on
    128-byte lines, and a stride that is a multiple of 1024 elements gets 64 more."""
    import torch
    from nlearn_amd.kernels.gemm import padded_empty

    cases = {(3, 12): 16, (3, 512): 512, (3, 1000): 1000, (3, 1536): 1536, (3, 2048): 2112, (3, 4096): 4160,
             (3, 2040): 2112, (3, 50257): 50304}
    for (r, c), ld in cases.items():
        t = padded_empty(r, c, torch.bfloat16, "cpu")
        assert t.shape == (r, c) and t.stride() == (ld, 1), (c, t.stride())
