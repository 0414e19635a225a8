"""CPU pins of the training-step oracle (oracle/model_np.py).

The NumPy forward/backward is checked against float64 torch autograd of the
same network written independently here (small configuration, no bf16
rounding), AdamW against its closed form, and the schedule against optax's
published formula at known points.
"""
import math

import numpy as np
import pytest
import torch

from oracle import model_np as om


def _torch_loss(params, batch, cfg):
    """Independent float64 restatement in torch (autograd supplies the backward)."""
    ids = torch.from_numpy(batch[:, :-1]).long()
    tg = torch.from_numpy(batch[:, 1:]).long()
    bs, S = ids.shape
    d, H = cfg.d, cfg.heads
    dh = d // H
    E = params["embeddings"]
    x = E["token_embed"][ids] + E["pos_embed"][:S]
    for b in params["blocks"]:
        h = torch.nn.functional.layer_norm(x, (d,), b["ln1"]["gamma"], b["ln1"]["beta"], cfg.eps)
        qkv = (h @ b["attn"]["W_qkv"]).view(bs, S, 3, H, dh)
        q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
        att = (q @ k.transpose(-1, -2)) / math.sqrt(dh)
        att = att.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf")).softmax(-1)
        o = (att @ v).transpose(1, 2).reshape(bs, S, d)
        x = x + o @ b["attn"]["W_o"]
        h2 = torch.nn.functional.layer_norm(x, (d,), b["ln2"]["gamma"], b["ln2"]["beta"], cfg.eps)
        u = torch.nn.functional.gelu(h2 @ b["ffn"]["W1"] + b["ffn"]["b1"], approximate="tanh")
        x = x + u @ b["ffn"]["W2"] + b["ffn"]["b2"]
    hf = torch.nn.functional.layer_norm(x, (d,), params["ln_final"]["gamma"], params["ln_final"]["beta"], cfg.eps)
    logits = hf @ params["lm_head"]
    return torch.nn.functional.cross_entropy(logits.reshape(-1, cfg.vocab), tg.reshape(-1))


def test_forward_backward_matches_float64_autograd():
    cfg = om.Config(vocab=97, d=32, heads=4, layers=2, ff=64, max_seq=16)
    p32 = om.init_params(3, cfg)
    rng = np.random.default_rng(0)
    # non-trivial LayerNorm parameters and biases so every gradient path is exercised
    for b in p32["blocks"]:
        for ln in ("ln1", "ln2"):
            b[ln]["gamma"] += rng.standard_normal(32).astype(np.float32) * 0.1
            b[ln]["beta"] += rng.standard_normal(32).astype(np.float32) * 0.1
        b["ffn"]["b1"] += rng.standard_normal(64).astype(np.float32) * 0.1
        b["ffn"]["b2"] += rng.standard_normal(32).astype(np.float32) * 0.1
    p64 = om._map(lambda a: a.astype(np.float64), p32)
    batch = rng.integers(0, cfg.vocab, (3, 13)).astype(np.int64)
    loss, grads = om.loss_and_grads(p64, batch, cfg, exact=True)
    tp = om._map(lambda a: torch.from_numpy(a.copy()).requires_grad_(True), p64)
    tl = _torch_loss(tp, batch, cfg)
    tl.backward()
    assert abs(loss - tl.item()) < 1e-10
    for g, t in zip(om._leaves(grads), om._leaves(tp)):
        np.testing.assert_allclose(g, t.grad.numpy(), rtol=1e-7, atol=1e-10)


def test_rounded_forward_stays_close_to_exact():
    cfg = om.Config(vocab=97, d=32, heads=4, layers=2, ff=64, max_seq=16)
    p = om.init_params(1, cfg)
    batch = np.random.default_rng(1).integers(0, cfg.vocab, (2, 9))
    l_exact, _ = om.loss_and_grads(p, batch, cfg, exact=True)
    l_bf16, _ = om.loss_and_grads(p, batch, cfg)
    assert abs(l_exact - l_bf16) < 5e-3
    assert abs(l_exact - math.log(cfg.vocab)) < 0.1   # tiny weights -> near-uniform prediction


def test_adamw_closed_form_first_steps():
    p = {"w": np.array([1.0], np.float64)}
    opt = om.AdamWNP(p, lambda c: 0.1, wd=0.5)
    g = {"w": np.array([2.0])}
    opt.step(p, g)
    # step 1: m = .1 g, v = .001 g^2, mhat = g, vhat = g^2 -> update sign(g) + wd * p
    assert p["w"][0] == pytest.approx(1.0 - 0.1 * (2.0 / (2.0 + 1e-8) + 0.5 * 1.0), rel=1e-12)


def test_adamw_constant_gradient_closed_form_every_step():
    """With a constant gradient g, m_t = (1 - b1^t) g and v_t = (1 - b2^t) g^2,
    so the bias-corrected moments are g and g^2 at EVERY t and each update is
    lr_t * (g / (|g| + eps) + wd * p). A bias correction frozen at t = 1 (or a
    count that does not advance) moves the t >= 2 updates off this."""
    lrs = [0.1, 0.05, 0.02, 0.3, 0.01]
    p = {"a": np.array([1.0, -2.0], np.float64), "b": np.array([[0.5]], np.float64)}
    g = {"a": np.array([3.0, -0.25]), "b": np.array([[1e-3]])}
    opt = om.AdamWNP(p, lambda c: lrs[c], wd=0.2)
    want = {k: v.copy() for k, v in p.items()}
    for t in range(len(lrs)):
        opt.step(p, g)
        for k in want:
            want[k] = want[k] - lrs[t] * (g[k] / (np.abs(g[k]) + 1e-8) + 0.2 * want[k])
            np.testing.assert_allclose(p[k], want[k], rtol=1e-12, atol=1e-15, err_msg=f"update {t + 1}, leaf {k}")


def test_adamw_second_and_third_updates_by_hand():
    """Changing gradients: the moments and bias corrections written out by
    hand for t = 2 and t = 3 (optax.adamw, train.py:504-505)."""
    b1, b2, eps, wd = 0.9, 0.999, 1e-8, 0.1
    g1, g2, g3 = 2.0, -0.5, 0.75
    lr = {0: 0.1, 1: 0.04, 2: 0.07}
    p = {"w": np.array([1.5], np.float64)}
    opt = om.AdamWNP(p, lambda c: lr[c], wd=wd)
    w = 1.5
    # t = 1
    opt.step(p, {"w": np.array([g1])})
    w = w - lr[0] * (g1 / (abs(g1) + eps) + wd * w)
    assert p["w"][0] == pytest.approx(w, rel=1e-13)
    # t = 2: m = b1 (1-b1) g1 + (1-b1) g2, v = b2 (1-b2) g1^2 + (1-b2) g2^2
    opt.step(p, {"w": np.array([g2])})
    m2 = b1 * (1 - b1) * g1 + (1 - b1) * g2
    v2 = b2 * (1 - b2) * g1 ** 2 + (1 - b2) * g2 ** 2
    w = w - lr[1] * ((m2 / (1 - b1 ** 2)) / (math.sqrt(v2 / (1 - b2 ** 2)) + eps) + wd * w)
    assert p["w"][0] == pytest.approx(w, rel=1e-13)
    # t = 3
    opt.step(p, {"w": np.array([g3])})
    m3 = b1 ** 2 * (1 - b1) * g1 + b1 * (1 - b1) * g2 + (1 - b1) * g3
    v3 = b2 ** 2 * (1 - b2) * g1 ** 2 + b2 * (1 - b2) * g2 ** 2 + (1 - b2) * g3 ** 2
    w = w - lr[2] * ((m3 / (1 - b1 ** 3)) / (math.sqrt(v3 / (1 - b2 ** 3)) + eps) + wd * w)
    assert p["w"][0] == pytest.approx(w, rel=1e-13)
    assert opt.count == 3


def test_adamw_clipped_second_update_by_hand():
    """optax.chain(clip_by_global_norm(1), adamw): update 1 below the threshold
    passes g untouched; update 2's global norm over both leaves is 5, so the
    gradient enters the moments as g * 1/5 (train.py:502-506)."""
    b1, b2, eps, wd = 0.9, 0.999, 1e-8, 0.1
    p = {"a": np.array([1.0], np.float64), "b": np.array([2.0], np.float64)}
    opt = om.AdamWNP(p, lambda c: 0.05, wd=wd, clip_norm=1.0)
    ga1, gb1 = 0.3, -0.4            # norm 0.5 < 1: unclipped
    ga2, gb2 = 3.0, 4.0             # norm 5 >= 1: scaled to (0.6, 0.8)
    opt.step(p, {"a": np.array([ga1]), "b": np.array([gb1])})
    opt.step(p, {"a": np.array([ga2]), "b": np.array([gb2])})
    for w0, g1, g2, k in ((1.0, ga1, ga2 / 5, "a"), (2.0, gb1, gb2 / 5, "b")):
        w = w0 - 0.05 * (g1 / (abs(g1) + eps) + wd * w0)
        m2 = b1 * (1 - b1) * g1 + (1 - b1) * g2
        v2 = b2 * (1 - b2) * g1 ** 2 + (1 - b2) * g2 ** 2
        w = w - 0.05 * ((m2 / (1 - b1 ** 2)) / (math.sqrt(v2 / (1 - b2 ** 2)) + eps) + wd * w)
        assert p[k][0] == pytest.approx(w, rel=1e-12), k


def test_multisteps_k2_by_hand():
    """optax.MultiSteps(adamw, 2): parameters unchanged on odd calls; the even
    call applies AdamW to the mean of the two micro-gradients, and the
    schedule count advances once per update (train.py:319-325,507-508)."""
    b1, b2, eps, wd = 0.9, 0.999, 1e-8, 0.1
    lr = {0: 0.1, 1: 0.02}
    p = {"w": np.array([1.0], np.float64)}
    ms = om.MultiStepsNP(om.AdamWNP(p, lambda c: lr[c], wd=wd), 2)
    ms.step(p, {"w": np.array([1.0])})
    assert p["w"][0] == 1.0
    ms.step(p, {"w": np.array([3.0])})          # mean 2
    w = 1.0 - lr[0] * (2.0 / (2.0 + eps) + wd * 1.0)
    assert p["w"][0] == pytest.approx(w, rel=1e-13)
    ms.step(p, {"w": np.array([-1.0])})
    assert p["w"][0] == pytest.approx(w, rel=1e-13)
    ms.step(p, {"w": np.array([0.0])})          # mean -0.5
    m2 = b1 * (1 - b1) * 2.0 + (1 - b1) * -0.5
    v2 = b2 * (1 - b2) * 4.0 + (1 - b2) * 0.25
    w = w - lr[1] * ((m2 / (1 - b1 ** 2)) / (math.sqrt(v2 / (1 - b2 ** 2)) + eps) + wd * w)
    assert p["w"][0] == pytest.approx(w, rel=1e-13)
    assert ms.inner.count == 2


def test_warmup_cosine_schedule_known_points():
    f = lambda c: om.warmup_cosine(c, 1e-3, 200, 1000, 1e-4)
    assert f(0) == 0.0
    assert f(100) == pytest.approx(5e-4)
    assert f(200) == pytest.approx(1e-3)
    assert f(600) == pytest.approx(1e-4 + 0.9e-3 * 0.5)      # half way down the cosine
    assert f(1000) == pytest.approx(1e-4)
    assert f(5000) == pytest.approx(1e-4)


def test_device_schedule_matches_oracle_schedule():
    from nlearn_amd.train import warmup_cosine_decay_schedule

    s = warmup_cosine_decay_schedule(0.0, 1e-3, 200, 1000, 1e-4)
    for c in (0, 1, 57, 199, 200, 201, 555, 999, 1000, 1234):
        assert s(c) == pytest.approx(om.warmup_cosine(c, 1e-3, 200, 1000, 1e-4), rel=1e-12, abs=1e-15)


def test_init_matches_device_initialiser():
    from nlearn_amd.model import ModelConfig, init_params_numpy, tree_leaves

    cfg = ModelConfig(vocab_size=97, d_model=32, n_heads=4, n_layers=2, d_ff=64, max_seq_len=16)
    a = tree_leaves(init_params_numpy(5, cfg))
    b = om._leaves(om.init_params(5, om.Config(vocab=97, d=32, heads=4, layers=2, ff=64, max_seq=16)))
    assert len(a) == len(b)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


def test_clip_by_global_norm_closed_form():
    """optax.clip_by_global_norm: the norm over all leaves; below the threshold
    the gradients pass unchanged, above it they are rescaled to norm max_norm
    with their direction kept."""
    from oracle import model_np as om

    rng = np.random.default_rng(5)
    g = {"a": rng.standard_normal((3, 4)).astype(np.float32), "b": [rng.standard_normal(7).astype(np.float32)]}
    flat = np.concatenate([g["a"].ravel(), g["b"][0]]).astype(np.float64)
    n = np.linalg.norm(flat)
    assert abs(om.global_norm(g) - n) < 1e-9 * n
    same = om.clip_by_global_norm(g, n * 1.01)
    assert same is g
    c = om.clip_by_global_norm(g, 0.5)
    cf = np.concatenate([c["a"].ravel(), c["b"][0]]).astype(np.float64)
    assert abs(np.linalg.norm(cf) - 0.5) < 1e-6
    np.testing.assert_allclose(cf * n / 0.5, flat, rtol=1e-6)


def test_multisteps_is_adamw_on_the_mean_gradient():
    """optax.MultiSteps(k=3): parameters unchanged on the first two calls; the
    third applies AdamW to the mean of the three gradients (the running mean
    acc + (g - acc)/(i+1) equals it up to rounding); the schedule count moves
    once per update."""
    from oracle import model_np as om

    rng = np.random.default_rng(6)
    p0 = {"w": rng.standard_normal((5, 6)).astype(np.float32), "v": rng.standard_normal(9).astype(np.float32)}
    gs = [{k: rng.standard_normal(x.shape).astype(np.float32) for k, x in p0.items()} for _ in range(6)]
    sched = lambda c: 1e-2 * (c + 1)  # noqa: E731
    pa = {k: x.copy() for k, x in p0.items()}
    ms = om.MultiStepsNP(om.AdamWNP(pa, sched), 3)
    pb = {k: x.copy() for k, x in p0.items()}
    ref = om.AdamWNP(pb, sched)
    for i, g in enumerate(gs):
        ms.step(pa, g)
        if i % 3 != 2:
            assert all(np.array_equal(pa[k], (p0 if i < 3 else pb)[k]) for k in p0)
        else:
            mean = {k: (gs[i - 2][k] + gs[i - 1][k] + gs[i][k]) / np.float32(3) for k in p0}
            ref.step(pb, mean)
            for k in p0:
                np.testing.assert_allclose(pa[k], pb[k], rtol=1e-5, atol=1e-7)
    assert ms.inner.count == 2 and ref.count == 2
