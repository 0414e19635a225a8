"""The allocation-free flash backward (nl_flash_attention_bwd_noalloc) against
nl_flash_attention_bwd with a caller workspace, through the C ABI.

Both run the same kernels over the same inputs, so dQ, dK and dV must be equal
bit for bit. Two calls in a row, the second smaller, check that the fixed
scratch array carries nothing from one call to the next; a size above
NL_FLASH_BWD_NOALLOC_MAX_ROWS must be refused before anything is launched.
"""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAX_ROWS = 2097152  # NL_FLASH_BWD_NOALLOC_MAX_ROWS in include/nlearn_hip.h


def _case(dev, B, H, S, seed):
    import torch

    g = torch.Generator(device="cpu").manual_seed(seed)
    q, k, v, do = (torch.randn((B, H, S, 64), generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
    return q, k, v, do


def _bwd_both(dev, q, k, v, do):
    import torch
    from nlearn_amd import _lib
    from nlearn_amd.attention import _stride4, flash_fwd_raw4

    B, H, S, D = q.shape
    scale = 1.0 / math.sqrt(D)
    O, L = flash_fwd_raw4(q, k, v)
    stream = torch.cuda.current_stream(dev).cuda_stream
    outs = []
    for noalloc in (False, True):
        dq, dk, dv = (torch.full((B, H, S, D), float("nan"), dtype=torch.bfloat16, device=dev) for _ in range(3))
        args = [stream, B, H, S, D, scale, 1,
                q.data_ptr(), _stride4(q), k.data_ptr(), _stride4(k), v.data_ptr(), _stride4(v),
                O.data_ptr(), _stride4(O), do.data_ptr(), _stride4(do), L.data_ptr(),
                dq.data_ptr(), _stride4(dq), dk.data_ptr(), _stride4(dk), dv.data_ptr(), _stride4(dv)]
        if noalloc:
            _lib.call("nl_flash_attention_bwd_noalloc", *args)
        else:
            ws = torch.empty(_lib.ws_bytes(B, H, S) // 4, dtype=torch.float32, device=dev)
            _lib.call("nl_flash_attention_bwd", *args, ws.data_ptr())
        outs.append((dq, dk, dv))
    torch.cuda.synchronize()
    return outs


def test_noalloc_backward_equals_workspace_backward_twice(dev):
    import torch

    # the second call is smaller: any stale D of the first would change it
    for B, H, S, seed in ((4, 8, 512, 11), (2, 3, 200, 12)):
        print(f"noalloc flash bwd B={B} H={H} S={S} seed={seed}", flush=True)
        q, k, v, do = _case(dev, B, H, S, seed)
        (a, b) = _bwd_both(dev, q, k, v, do)
        for name, x, y in zip(("dQ", "dK", "dV"), a, b):
            assert torch.isfinite(y.float()).all(), name
            assert torch.equal(x, y), (name, B, H, S)


def test_noalloc_backward_refuses_oversize(dev):
    from nlearn_amd import _lib

    lib = _lib.load()
    s = _lib.AttnStride(0, 0, 64)
    # batch*heads*seq = MAX_ROWS + 64: refused on the host, nothing launched
    rc = lib.nl_flash_attention_bwd_noalloc(None, 1, 1, MAX_ROWS + 64, 64, 0.125, 1, 256, s, 256, s, 256, s,
                                            256, s, 256, s, 256, 256, s, 256, s, 256, s)
    assert rc == _lib.NL_EINVAL
    assert b"NL_FLASH_BWD_NOALLOC_MAX_ROWS" in lib.nl_last_error()
