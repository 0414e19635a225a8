"""The fused AdamW kernels against the optax.adamw restatement, element-wise.

oracle.model_np.AdamWNP follows optax.adamw as the reference calls it
(train.py:504-505): bias-corrected Adam moments, decoupled decay lr*wd*p on
every leaf, lr from the schedule at the pre-update count. Here it runs in
float64 on the same gradients. Both device paths are checked for three
updates with a changing lr: one launch over the whole tree (nl_adamw_multi,
gradients in main_grad) and one launch per leaf (nl_adamw_step, .grad). The
leaves include the LM head's padded layout (50257 columns stored with row
stride 50264; the padding must stay zero) and bf16 shadows, which must hold
the round-to-nearest-even bf16 of the updated fp32 weight.
"""
import numpy as np
import pytest

from oracle import model_np as om
from oracle import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("multi", [True, False], ids=["nl_adamw_multi", "nl_adamw_step"])
def test_adamw_matches_oracle_elementwise(dev, multi):
    import torch
    from nlearn_amd.kernels.gemm import bf16_shadow
    from nlearn_amd.model import device_param
    from nlearn_amd.train import AdamW

    shapes = {"head": (512, 50257), "vec": (7,), "w": (64, 2048), "odd": (8193,), "row": (1, 12)}
    rng = np.random.default_rng(81)
    init = {k: (rng.standard_normal(s) * 0.02).astype(np.float32) for k, s in shapes.items()}
    params = {k: device_param(v, dev) for k, v in init.items()}
    assert params["head"].stride(0) == 50264
    sched = lambda c: 1e-3 * (c + 1)  # noqa: E731  lr changes every update
    opt = AdamW(sched, weight_decay=0.1, grad_buffers=multi)
    state = opt.init(params)
    for k in ("head", "w"):
        bf16_shadow(params[k])
    ref_p = {k: v.astype(np.float64) for k, v in init.items()}
    ref = om.AdamWNP(ref_p, sched, wd=0.1)
    for step in range(3):
        grads = {k: rng.standard_normal(s).astype(np.float32) for k, s in shapes.items()}
        for k, p in params.items():
            g = torch.from_numpy(grads[k]).to(dev)
            if multi:
                p.main_grad.copy_(g)
            else:
                p.grad = g
        with torch.no_grad():
            opt.update(params, state)
        ref.step(ref_p, {k: g.astype(np.float64) for k, g in grads.items()})
        torch.cuda.synchronize()
        for i, k in enumerate(shapes):
            p = params[k].detach().cpu().numpy()
            # fp32 against float64: a few ulps of the weights' scale (ulp(0.03) = 3.7e-9) per update
            np.testing.assert_allclose(p, ref_p[k], rtol=1e-5, atol=2e-8, err_msg=f"p {k} step {step}")
            # m = 0.9 m + 0.1 g cancels near zero: a few ulps of its terms (|0.1 g| < 0.6, ulp 6e-8)
            np.testing.assert_allclose(state["mu"][i].cpu().numpy(), ref.m[i], rtol=1e-5, atol=2e-7,
                                       err_msg=f"m {k} step {step}")
            # v's terms are positive (no cancellation); values ~1e-3 g^2
            np.testing.assert_allclose(state["nu"][i].cpu().numpy(), ref.v[i], rtol=1e-5, atol=1e-10,
                                       err_msg=f"v {k} step {step}")
        head = params["head"].detach()
        full = torch.as_strided(head, (512, 50264), (50264, 1))
        assert torch.count_nonzero(full[:, 50257:]).item() == 0
        for k in ("head", "w"):
            sh = params[k]._nl_bf16
            bits = sh.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
            want = ops.bf16_bits(params[k].detach().cpu().numpy())
            assert np.array_equal(bits, want), k
