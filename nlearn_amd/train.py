"""nlearn_amd.train — the training step around the HIP kernels (mirrors nlearn/train.py).

* ``batch_loss(params, batch)``      mean next-token CE of a (bs, seq+1) batch
                                     (train.py:270-299, the batched fused-CE path)
* ``warmup_cosine_decay_schedule``   optax's schedule (train.py:487-495)
* ``AdamW``                          optax.adamw semantics (train.py:504-505) on the
                                     fused HIP kernel; writes the bf16 weight shadows
* ``make_train_step(optimizer)``     value_and_grad + update (train.py:328-341)
* ``train(...)``                     offline loop on a synthetic uniform token stream
                                     (train.py:482-622 streams a HF corpus instead)

``python -m nlearn_amd.train --steps N`` runs offline: no dataset download, no
tokenizer, no wandb (the reference needs all three, train.py:433-443,515-535).
"""
from __future__ import annotations

import argparse
import math
import os
import time

import torch

from . import _lib
from .kernels.cross_entropy import cross_entropy
from .model import BASELINE, ModelConfig, count_params, init_model, model_forward, tree_leaves

WARMUP_STEPS = int(os.environ.get("NLEARN_WARMUP", "200"))
PEAK_LR = 1e-3
WEIGHT_DECAY = float(os.environ.get("NLEARN_WD", "0.1"))
BATCH_SIZE = 32


# ---------------------------------------------------------------------------
# loss
# ---------------------------------------------------------------------------


def batch_loss(params, batch: torch.Tensor, cfg: ModelConfig = BASELINE) -> torch.Tensor:
    """Mean CE of predicting batch[:, 1:] from batch[:, :-1] (train.py:270-285).

    The logits are only read by the CE, so its single pass writes dlogits over
    them (inplace=True): the (bs*seq, vocab) gradient costs no extra memory.
    """
    input_ids = batch[:, :-1]
    target_ids = batch[:, 1:]
    logits = model_forward(params, input_ids, cfg)
    return cross_entropy(logits, target_ids, inplace=True)


# ---------------------------------------------------------------------------
# optimizer
# ---------------------------------------------------------------------------


def warmup_cosine_decay_schedule(init_value: float, peak_value: float, warmup_steps: int, decay_steps: int,
                                 end_value: float):
    """optax.warmup_cosine_decay_schedule: linear 0->peak over warmup_steps, then
    cosine peak->end until decay_steps (measured from step 0)."""

    def schedule(count: int) -> float:
        if warmup_steps > 0 and count < warmup_steps:
            return init_value + (peak_value - init_value) * count / warmup_steps
        span = max(decay_steps - warmup_steps, 1)
        t = min(max(count - warmup_steps, 0), span) / span
        return end_value + (peak_value - end_value) * 0.5 * (1.0 + math.cos(math.pi * t))

    return schedule


class AdamW:
    """optax.adamw(learning_rate=schedule, b1=.9, b2=.999, eps=1e-8, weight_decay)
    with decoupled decay on every parameter. The schedule is evaluated at the
    update count before the update (optax's ``count``), bias corrections use the
    count after it."""

    def __init__(self, learning_rate, weight_decay: float = WEIGHT_DECAY, b1: float = 0.9, b2: float = 0.999,
                 eps: float = 1e-8):
        self.lr = learning_rate if callable(learning_rate) else (lambda _c, v=learning_rate: v)
        self.wd, self.b1, self.b2, self.eps = weight_decay, b1, b2, eps

    def init(self, params) -> dict:
        leaves = tree_leaves(params)
        return {"count": 0,
                "mu": [torch.zeros_like(p, dtype=torch.float32) for p in leaves],
                "nu": [torch.zeros_like(p, dtype=torch.float32) for p in leaves]}

    def update(self, params, state: dict) -> dict:
        """Apply one step in place using each parameter's ``.grad``."""
        count = state["count"]
        lr = float(self.lr(count))
        t = count + 1
        bc1, bc2 = 1.0 - self.b1 ** t, 1.0 - self.b2 ** t
        for p, m, v in zip(tree_leaves(params), state["mu"], state["nu"]):
            g = p.grad
            if g is None:
                continue
            if not g.is_contiguous():
                g = g.contiguous()
            shadow = getattr(p, "_nl_bf16", None)
            rows = p.shape[0] if p.dim() == 2 else 1
            cols = p.shape[1] if p.dim() == 2 else p.numel()
            sb, ldb = (None, 0)
            if shadow is not None and getattr(p, "_nl_bf16_version", None) == p._version:
                sb, ldb = shadow.data_ptr(), (shadow.stride(0) if shadow.dim() == 2 else cols)
            _lib.call("nl_adamw_step", torch.cuda.current_stream(p.device).cuda_stream, rows, cols,
                      p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), sb, ldb, lr, self.b1, self.b2,
                      self.eps, self.wd, bc1, bc2)
        state["count"] = t
        return state


def make_train_step(optimizer: AdamW, cfg: ModelConfig = BASELINE):
    """train_step(params, opt_state, batch) -> (params, opt_state, loss).

    Parameters are updated in place; the loss is a 0-d device tensor (no host
    sync inside the step, as with the jitted step of train.py:328-341).
    """

    def train_step(params, opt_state, batch):
        leaves = tree_leaves(params)
        for p in leaves:
            p.grad = None
        loss = batch_loss(params, batch, cfg)
        loss.backward()
        with torch.no_grad():
            opt_state = optimizer.update(params, opt_state)
        return params, opt_state, loss.detach()

    return train_step


# ---------------------------------------------------------------------------
# data + loop
# ---------------------------------------------------------------------------


class SyntheticTokens:
    """Uniform random token stream of (bs, seq+1) int32 batches, seeded."""

    def __init__(self, bs: int, seq: int, vocab: int, seed: int = 0, device="cuda"):
        self.bs, self.seq, self.vocab = bs, seq, vocab
        self.gen = torch.Generator(device=device).manual_seed(seed)
        self.device = device

    def get_batch(self) -> torch.Tensor:
        return torch.randint(0, self.vocab, (self.bs, self.seq + 1), generator=self.gen, device=self.device,
                             dtype=torch.int32)


def train(steps: int = 20, seq_len: int = 512, seed: int = 0, batch_size: int = BATCH_SIZE,
          peak_lr: float = PEAK_LR, log_every: int = 10, cfg: ModelConfig | None = None) -> list:
    """Offline training loop; returns the per-step losses."""
    cfg = cfg or ModelConfig(max_seq_len=max(seq_len, BASELINE.max_seq_len))
    warmup = min(WARMUP_STEPS, max(1, steps) // 5)
    sched = warmup_cosine_decay_schedule(0.0, peak_lr, warmup, max(1, steps), peak_lr / 10)
    opt = AdamW(sched)
    params = init_model(seed, cfg)
    print(f"params: {count_params(params) / 1e6:.1f} M  bs={batch_size} seq={seq_len} warmup={warmup}")
    state = opt.init(params)
    step_fn = make_train_step(opt, cfg)
    data = SyntheticTokens(batch_size, seq_len, cfg.vocab_size, seed)
    losses = []
    t0 = time.time()
    for i in range(steps):
        params, state, loss = step_fn(params, state, data.get_batch())
        losses.append(loss)
        if (i + 1) % log_every == 0 or i + 1 == steps:
            torch.cuda.synchronize()
            dt = time.time() - t0
            print(f"step {i + 1:5d}  loss {loss.item():.4f}  {(i + 1) * batch_size * seq_len / dt:,.0f} tok/s")
    return [float(l) for l in torch.stack(losses).cpu()]


def main(argv=None):
    ap = argparse.ArgumentParser(description="offline nlearn training on the HIP kernels")
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--seq-len", type=int, default=512)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--batch-size", type=int, default=BATCH_SIZE)
    ap.add_argument("--peak-lr", type=float, default=PEAK_LR)
    a = ap.parse_args(argv)
    train(a.steps, a.seq_len, a.seed, a.batch_size, a.peak_lr)


if __name__ == "__main__":
    main()
