"""The LM head + cross-entropy with the CE of each row chunk pipelined behind
the next chunk's logits GEMM (kernels.cross_entropy.lm_head_cross_entropy)
must equal the unchunked linear + cross_entropy bit for bit: loss, dX and dW."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,d,V,chunks,g", [(37, 64, 1000, 3, 1.0), (1024, 512, 5000, 4, 3.0),
                                            (1000, 512, 50257, 7, 1.0), (16384, 512, 50257, 4, 1.0),
                                            (16384, 512, 50257, 2, 2.0), (3000, 512, 50257, 2, 1.0)])
def test_lm_head_cross_entropy_equals_linear_then_ce(dev, M, d, V, chunks, g):
    import torch
    from nlearn_amd.kernels.cross_entropy import cross_entropy, lm_head_cross_entropy
    from nlearn_amd.kernels.gemm import linear

    rng = np.random.default_rng(M + V + chunks)
    X = torch.from_numpy(rng.standard_normal((M, d)).astype(np.float32) * 0.5).to(dev).bfloat16()
    W = torch.from_numpy(rng.standard_normal((d, V)).astype(np.float32) * 0.05).to(dev)
    t = torch.from_numpy(rng.integers(0, V, M).astype(np.int32)).to(dev)
    out = {}
    for path in ("reference", "chunked"):
        Xp = X.clone().requires_grad_(True)
        Wp = W.clone().requires_grad_(True)
        if path == "reference":
            loss = cross_entropy(linear(Xp, Wp), t, inplace=True)
        else:
            loss = lm_head_cross_entropy(Xp, Wp, t, chunks)
        (loss * g).backward()
        torch.cuda.synchronize()
        out[path] = (loss.detach(), Xp.grad, Wp.grad)
    (l1, dx1, dw1), (l2, dx2, dw2) = out["reference"], out["chunked"]
    assert torch.isfinite(l1) and float(l1) > 0
    assert torch.equal(l1, l2)
    assert torch.equal(dx1, dx2)
    assert torch.equal(dw1, dw2)


def test_lm_head_cross_entropy_single_chunk_and_more_chunks_than_rows(dev):
    import torch
    from nlearn_amd.kernels.cross_entropy import lm_head_cross_entropy

    rng = np.random.default_rng(5)
    X = torch.from_numpy(rng.standard_normal((3, 64)).astype(np.float32)).to(dev).bfloat16()
    W = torch.from_numpy(rng.standard_normal((64, 300)).astype(np.float32) * 0.1).to(dev)
    t = torch.from_numpy(rng.integers(0, 300, 3).astype(np.int32)).to(dev)
    losses = [lm_head_cross_entropy(X, W, t, c) for c in (1, 2, 3, 16)]
    torch.cuda.synchronize()
    for other in losses[1:]:
        assert torch.equal(losses[0], other)
    with pytest.raises(ValueError):
        lm_head_cross_entropy(X, W, t[:2], 2)
