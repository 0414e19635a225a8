"""The captured training step and the multi-tensor AdamW against their eager forms.

* nl_adamw_multi (one launch over the whole tree, scalars read from device
  memory) must equal nl_adamw_step per leaf bit for bit: same arithmetic.
* Weight gradients written into the optimizer's main_grad buffers equal the
  ones autograd returns without buffers, bit for bit (every kernel of the step
  sums in a fixed order, the token-embedding gradient included).
* The HIP-graph step replayed several times, with eager work and host
  synchronisations between replays, gives the eager step's losses and
  parameters bit for bit.
"""
import numpy as np
import pytest


pytestmark = pytest.mark.gpu


def test_adamw_multi_matches_per_leaf(dev):
    import torch
    from nlearn_amd.model import device_param
    from nlearn_amd.train import AdamW, attach_grad_buffers
    from nlearn_amd.kernels.gemm import bf16_shadow

    rng = np.random.default_rng(0)
    shapes = [(512, 50257), (7,), (3, 5), (64, 2048), (1, 12), (8193,)]

    def make():
        params = {f"p{i}": device_param(rng.standard_normal(s).astype(np.float32), dev) for i, s in enumerate(shapes)}
        return params

    rng = np.random.default_rng(0)
    pa = make()
    rng = np.random.default_rng(0)
    pb = make()
    grads = [np.random.default_rng(10 + i).standard_normal(s).astype(np.float32) for i, s in enumerate(shapes)]
    sched = lambda c: 1e-2 * (c + 1)
    oa, ob = AdamW(sched, grad_buffers=True), AdamW(sched, grad_buffers=False)
    sa, sb = oa.init(pa), ob.init(pb)
    for k in ("p0", "p3"):       # GEMM weights carry bf16 shadows
        bf16_shadow(pa[k])
        bf16_shadow(pb[k])
    for step in range(3):
        for (ka, a), (kb, b), g in zip(pa.items(), pb.items(), grads):
            gt = torch.from_numpy(g * (step + 1)).to(dev)
            a.main_grad.copy_(gt)
            b.grad = gt.clone()
        with torch.no_grad():
            oa.update(pa, sa)
            ob.update(pb, sb)
        torch.cuda.synchronize()
        assert sa["table"] is not None
        for k in pa:
            assert torch.equal(pa[k], pb[k]), (step, k)
        for ma, mb in zip(sa["mu"] + sa["nu"], sb["mu"] + sb["nu"]):
            assert torch.equal(ma, mb)
        for k in ("p0", "p3"):
            assert torch.equal(pa[k]._nl_bf16, pb[k]._nl_bf16)
            assert torch.equal(pa[k]._nl_bf16, pa[k].detach().to(torch.bfloat16))


def test_main_grad_buffers_match_autograd(dev):
    import torch
    from nlearn_amd.model import ModelConfig, init_model, tree_leaves
    from nlearn_amd.train import attach_grad_buffers, batch_loss

    cfg = ModelConfig(max_seq_len=128)
    batch = torch.from_numpy(np.random.default_rng(3).integers(0, 50257, (2, 129)).astype(np.int32)).to(dev)
    pa = init_model(0, cfg, dev)
    pb = init_model(0, cfg, dev)
    attach_grad_buffers(pb)
    la = batch_loss(pa, batch, cfg)
    la.backward()
    lb = batch_loss(pb, batch, cfg)
    lb.backward()
    torch.cuda.synchronize()
    assert la.item() == lb.item()
    for i, (a, b) in enumerate(zip(tree_leaves(pa), tree_leaves(pb))):
        assert b.grad is None
        assert torch.equal(a.grad, b.main_grad), i


def test_graphed_step_matches_eager(dev):
    import torch
    from nlearn_amd.model import ModelConfig, init_model, tree_leaves
    from nlearn_amd.train import AdamW, make_train_step, warmup_cosine_decay_schedule

    cfg = ModelConfig(max_seq_len=128)
    rng = np.random.default_rng(9)
    batches = [torch.from_numpy(rng.integers(0, 50257, (2, 129)).astype(np.int32)).to(dev) for _ in range(8)]
    sched = warmup_cosine_decay_schedule(0.0, 1e-3, 3, 8, 1e-4)
    runs = {}
    for graph in (False, True):
        opt = AdamW(sched)
        params = init_model(0, cfg, dev)
        state = opt.init(params)
        step = make_train_step(opt, cfg, graph=graph, warmup=2)
        losses = []
        for i, b in enumerate(batches):
            params, state, loss = step(params, state, b)
            losses.append(loss)
            # unrelated eager work and a host sync between replays
            torch.cuda.synchronize()
            junk = torch.randn(1000, device=dev).sum()
            assert torch.isfinite(junk)
        torch.cuda.synchronize()
        runs[graph] = ([float(l) for l in losses], [p.detach().clone() for p in tree_leaves(params)], state["count"])
    (le, pe, ce), (lg, pg, cg) = runs[False], runs[True]
    assert ce == cg == 8
    assert lg == le
    assert len(set(lg)) == len(lg)          # every replay produced a fresh loss
    for a, b in zip(pe, pg):
        assert torch.equal(a, b)


@pytest.mark.parametrize("graph", [False, True], ids=["eager", "hip_graph"])
def test_overlapped_weight_grads_are_bit_identical(dev, graph):
    """Weight gradients forked onto a second stream (kernels.wgrad) change the
    schedule only: losses, parameters, moments and bf16 shadows after 4 steps
    equal the one-stream step bit for bit (a missed join or a buffer recycled
    under the side stream would show up as a difference)."""
    import torch
    from nlearn_amd.model import ModelConfig, init_model, tree_leaves
    from nlearn_amd.train import AdamW, make_train_step, warmup_cosine_decay_schedule

    cfg = ModelConfig(max_seq_len=128)
    rng = np.random.default_rng(21)
    batches = [torch.from_numpy(rng.integers(0, 50257, (2, 129)).astype(np.int32)).to(dev) for _ in range(4)]
    sched = warmup_cosine_decay_schedule(0.0, 1e-3, 2, 4, 1e-4)
    runs = {}
    for overlap in (False, True):
        opt = AdamW(sched)
        params = init_model(0, cfg, dev)
        state = opt.init(params)
        step = make_train_step(opt, cfg, graph=graph, warmup=1, overlap_wgrad=overlap)
        losses = []
        for b in batches:
            params, state, loss = step(params, state, b)
            losses.append(float(loss))
        torch.cuda.synchronize()
        leaves = tree_leaves(params)
        shadows = [sh.clone() for sh in (getattr(p, "_nl_bf16", None) for p in leaves) if sh is not None]
        runs[overlap] = (losses, [p.detach().clone() for p in leaves] + [t.clone() for t in state["mu"] + state["nu"]]
                         + shadows)
    assert runs[True][0] == runs[False][0]
    assert len(runs[True][1]) == len(runs[False][1])
    for a, b in zip(runs[False][1], runs[True][1]):
        assert torch.equal(a, b)
