"""Gradient accumulation (optax.MultiSteps), global-norm clipping and loss
scaling on the device, against their optax restatements in the oracle.

* nl_global_norm against the float64 norm of the whole gradient buffer.
* AdamW(clip_norm) (nl_global_norm + nl_adamw_multi_clip) element-wise
  against AdamWNP(clip_norm) over updates where the clip does and does not
  trigger (m and v scale with the clip factor, so they pin it).
* MultiSteps(AdamW, k=3) with a loss scale of 8 (gradients arrive scaled by
  8 and are divided on the device): the accumulated mean after every
  micro-step, and p, m, v after each update, against MultiStepsNP; the
  parameters do not move on the other micro-steps.
* The model: K = 4 micro-batches of bs8 give the update of one bs32 step
  (the mean of four micro-batch means is the bs32 mean), through the
  captured HIP graph; and a K = 2 run with clipping and loss scale 1024
  follows the oracle's loss curve.
"""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import model_np as om

pytestmark = pytest.mark.gpu

SHAPES = {"head": (512, 50257), "vec": (7,), "w": (64, 2048), "odd": (8193,)}


def _params(dev, seed):
    from nlearn_amd.model import device_param

    rng = np.random.default_rng(seed)
    init = {k: (rng.standard_normal(s) * 0.02).astype(np.float32) for k, s in SHAPES.items()}
    return init, {k: device_param(v, dev) for k, v in init.items()}


def _cmp(dev_t, ref, what, rtol=1e-5, atol=2e-8):
    np.testing.assert_allclose(dev_t.detach().cpu().numpy(), ref, rtol=rtol, atol=atol, err_msg=what)


def test_global_norm_matches_float64(dev):
    import torch
    from nlearn_amd import _lib

    rng = np.random.default_rng(90)
    for n in (1, 7, 4096, 3 * 1024 * 1024 + 5):
        x = rng.standard_normal(n).astype(np.float32)
        xd = torch.from_numpy(x).to(dev)
        out = torch.full((1,), float("nan"), device=dev)
        ws = torch.empty(int(_lib.load().nl_global_norm_ws_bytes(n)) // 4, device=dev)
        _lib.call("nl_global_norm", torch.cuda.current_stream().cuda_stream, n, xd.data_ptr(), out.data_ptr(),
                  ws.data_ptr(), ws.numel() * 4)
        torch.cuda.synchronize()
        ref = np.linalg.norm(x.astype(np.float64))
        assert abs(out.item() - ref) <= 1e-5 * ref, (n, out.item(), ref)


def test_adamw_clip_matches_oracle(dev):
    import torch
    from nlearn_amd.train import AdamW

    init, params = _params(dev, 91)
    sched = lambda c: 1e-3  # noqa: E731
    opt = AdamW(sched, clip_norm=40.0)
    state = opt.init(params)
    ref_p = {k: v.astype(np.float64) for k, v in init.items()}
    ref = om.AdamWNP(ref_p, sched, clip_norm=40.0)
    rng = np.random.default_rng(92)
    # global norms ~ sqrt(26.3M) * scale: 5128 * 0.02 = 103 (clipped), 5128 * 0.004 = 21 (not), then clipped
    for step, gscale in enumerate((0.02, 0.004, 0.05)):
        grads = {k: (rng.standard_normal(s) * gscale).astype(np.float32) for k, s in SHAPES.items()}
        for k, p in params.items():
            p.main_grad.copy_(torch.from_numpy(grads[k]))
        with torch.no_grad():
            opt.update(params, state)
        ref.step(ref_p, {k: g.astype(np.float64) for k, g in grads.items()})
        torch.cuda.synchronize()
        gn = om.global_norm(grads)
        assert abs(state["gnorm"].item() - gn) <= 1e-5 * gn
        for i, k in enumerate(SHAPES):
            _cmp(params[k], ref_p[k], f"p {k} step {step}")
            _cmp(state["mu"][i], ref.m[i], f"m {k} step {step}", atol=2e-7 * gscale / 0.02)
            _cmp(state["nu"][i], ref.v[i], f"v {k} step {step}", atol=1e-10)


def test_multisteps_with_loss_scale_matches_oracle(dev):
    import torch
    from nlearn_amd.train import AdamW, MultiSteps

    init, params = _params(dev, 93)
    sched = lambda c: 1e-3 * (c + 1)  # noqa: E731
    opt = MultiSteps(AdamW(sched, clip_norm=40.0), 3)
    state = opt.init(params)
    ref_p = {k: v.astype(np.float64) for k, v in init.items()}
    ref = om.MultiStepsNP(om.AdamWNP(ref_p, sched, clip_norm=40.0), 3)
    rng = np.random.default_rng(94)
    S = 8.0
    for step in range(6):
        grads = {k: (rng.standard_normal(s) * 0.02).astype(np.float32) for k, s in SHAPES.items()}
        before = {k: p.detach().clone() for k, p in params.items()}
        for k, p in params.items():       # the backward of a loss scaled by S
            p.main_grad.copy_(torch.from_numpy(grads[k] * np.float32(S)))
        with torch.no_grad():
            opt.update(params, state, loss_scale=S)
        # the running mean in fp32, the gradients' dtype (as optax forms it); Adam in float64
        ref.step(ref_p, grads)
        torch.cuda.synchronize()
        if step % 3 != 2:
            assert state["mini_step"] == step % 3 + 1
            for i, k in enumerate(SHAPES):
                assert torch.equal(params[k], before[k]), (step, k)
                _cmp(state["inner"]["grads"][i], ref.acc[k], f"acc {k} step {step}", atol=1e-8)
        else:
            assert state["mini_step"] == 0 and state["count"] == step // 3 + 1
            for i, k in enumerate(SHAPES):
                _cmp(params[k], ref_p[k], f"p {k} step {step}")
                _cmp(state["mu"][i], ref.inner.m[i], f"m {k} step {step}", atol=2e-7)
                _cmp(state["nu"][i], ref.inner.v[i], f"v {k} step {step}", atol=1e-10)


def test_model_k4_bs8_equals_one_bs32_step(dev):
    """K = 4 micro-batches of 8 sequences through the captured graph = one step
    on the 32 sequences: the same mean gradient (up to summation order) and
    the same update; the parameters are untouched on micro-steps 1-3."""
    import torch
    from nlearn_amd.model import init_model, tree_leaves
    from nlearn_amd.train import AdamW, MultiSteps, make_train_step

    rng = np.random.default_rng(95)
    big = torch.from_numpy(rng.integers(0, 50257, (32, 513)).astype(np.int32)).to(dev)
    pa = init_model(0, device=dev)
    p0 = [p.detach().clone() for p in tree_leaves(pa)]
    oa = MultiSteps(AdamW(lambda c: 1e-3), 4)
    sa = oa.init(pa)
    step_a = make_train_step(oa, graph=True, warmup=1)
    la = []
    for i in range(4):
        pa, sa, loss = step_a(pa, sa, big[8 * i:8 * i + 8].contiguous())
        la.append(loss.item())
        if i < 3:
            assert all(torch.equal(p, q) for p, q in zip(tree_leaves(pa), p0)), i
    pb = init_model(0, device=dev)
    ob = AdamW(lambda c: 1e-3)
    sb = ob.init(pb)
    _, _, lb = make_train_step(ob)(pb, sb, big)
    torch.cuda.synchronize()
    assert sa["count"] == 1 and sb["count"] == 1
    assert abs(np.mean(la) - lb.item()) < 1e-4
    # bf16 level: the GEMM plans differ between M = 4096 and 16384 (e.g. the
    # LM-head dX splits K 8 ways at bs8, 2 ways at bs32), and one fp32 rounding
    # of difference flips some bf16 roundings (2^-8); a wrong accumulation
    # (a sum, or one micro-batch) would be off by O(1)
    for i, (ga, pbl) in enumerate(zip(sa["inner"]["grads"], tree_leaves(pb))):
        assert rel_l2(ga.cpu().numpy(), pbl.main_grad.cpu().numpy(), floor=1e-8) < 2e-2, i
    # Adam's first update is ~ lr * sign(g): elements whose gradient cancels to
    # ~0 may flip between the two roundings, so compare update directions
    # (the update arithmetic itself is pinned element-wise above)
    for i, (a, b, z) in enumerate(zip(tree_leaves(pa), tree_leaves(pb), p0)):
        da, db = (a - z).detach(), (b - z).detach()
        agree = (torch.sign(da) == torch.sign(db)).float().mean().item()
        assert agree > 0.99, (i, agree)


def test_model_accum_clip_loss_scale_curve_matches_oracle(dev):
    """K = 2, clip_by_global_norm(0.5), loss scale 1024, 8 micro-steps at bs2 x
    seq128 through the HIP graph: the losses follow TrainStepNP with the same
    optimizer chain within 1e-2."""
    import torch
    from nlearn_amd.model import ModelConfig, init_model
    from nlearn_amd.train import AdamW, MultiSteps, make_train_step

    cfg = ModelConfig(max_seq_len=128)
    rng = np.random.default_rng(96)
    batches = [rng.integers(0, 50257, (2, 129)).astype(np.int32) for _ in range(8)]
    opt = MultiSteps(AdamW(lambda c: 1e-3, clip_norm=0.5), 2)
    params = init_model(0, cfg, dev)
    state = opt.init(params)
    step = make_train_step(opt, cfg, graph=True, loss_scale=1024.0)
    gpu = []
    for b in batches:
        params, state, loss = step(params, state, torch.from_numpy(b).to(dev))
        gpu.append(loss.item())
    assert state["count"] == 4
    assert state["inner"]["gnorm"].item() > 0.5      # the clip did trigger
    ocfg = om.Config(max_seq=128)
    ref = om.TrainStepNP(om.init_params(0, ocfg), lr=1e-3, warmup=0, decay_steps=0, cfg=ocfg, accum=2,
                         clip_norm=0.5)
    cpu = [ref(b.astype(np.int64)) for b in batches]
    print("gpu", np.round(gpu, 5).tolist(), "cpu", np.round(cpu, 5).tolist())
    assert np.abs(np.array(gpu) - np.array(cpu)).max() < 1e-2


def test_multisteps_resume_mid_accumulation(dev, tmp_path, monkeypatch):
    """save_resume_state after 3 micro-steps of MultiSteps(k = 2) (one update
    done, one micro-step accumulated), then load_resume_state into a fresh
    optimizer: the next micro-steps give the uninterrupted run's losses and
    parameters (the mini-step and the running mean travel in resume.pkl)."""
    import torch
    from nlearn_amd.model import ModelConfig, init_model, tree_leaves
    from nlearn_amd.train import AdamW, MultiSteps, load_resume_state, make_train_step, save_resume_state

    monkeypatch.chdir(tmp_path)
    cfg = ModelConfig(max_seq_len=64)
    rng = np.random.default_rng(97)
    batches = [torch.from_numpy(rng.integers(0, 50257, (2, 65)).astype(np.int32)).to(dev) for _ in range(6)]
    sched = lambda c: 1e-3  # noqa: E731
    opt = MultiSteps(AdamW(sched), 2)
    params = init_model(0, cfg, dev)
    state = opt.init(params)
    step = make_train_step(opt, cfg)
    for b in batches[:3]:
        params, state, _ = step(params, state, b)
    assert state["mini_step"] == 1 and state["count"] == 1
    save_resume_state(params, state, 3, run_name="ms")
    la = []
    for b in batches[3:]:
        params, state, loss = step(params, state, b)
        la.append(float(loss))
    opt2 = MultiSteps(AdamW(sched), 2)
    params2, state2, nxt = load_resume_state(opt2, run_name="ms", device=dev)
    assert nxt == 3 and state2["mini_step"] == 1 and state2["count"] == 1 and state2["inner"]["count"] == 1
    step2 = make_train_step(opt2, cfg)
    lb = []
    for b in batches[3:]:
        params2, state2, loss = step2(params2, state2, b)
        lb.append(float(loss))
    np.testing.assert_allclose(lb, la, rtol=1e-6, atol=1e-6)
    for a, c in zip(tree_leaves(params), tree_leaves(params2)):
        assert rel_l2(c.detach().cpu().numpy(), a.detach().cpu().numpy()) < 1e-5
