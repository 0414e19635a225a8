"""nlearn_amd.train — the training step around the HIP kernels (mirrors nlearn/train.py).

* ``batch_loss(params, batch)``      mean next-token CE of a (bs, seq+1) batch
                                     (train.py:270-299, the batched fused-CE path)
* ``warmup_cosine_decay_schedule``   optax's schedule (train.py:487-495)
* ``AdamW``                          optax.adamw semantics (train.py:504-505) on the
                                     fused HIP kernel; writes the bf16 weight shadows
* ``make_train_step(optimizer)``     value_and_grad + update (train.py:328-341)
* ``train(...)``                     offline loop on a synthetic uniform token stream
                                     (train.py:482-622 streams a HF corpus instead),
                                     with the reference's checkpoint / resume files
* ``save_checkpoint`` ... ``load_resume_state``  the checkpoint format (train.py:36-99;
                                     nlearn_amd.checkpoint)

``python -m nlearn_amd.train --steps N`` runs offline: no dataset download, no
tokenizer, no wandb (the reference needs all three, train.py:433-443,515-535).
"""
from __future__ import annotations

import argparse
import contextlib
import math
import os
import time

import torch

from . import _lib
from .checkpoint import load_checkpoint, load_resume_state, save_checkpoint, save_resume_state  # noqa: F401
from .kernels import fused, wgrad
from .kernels.cross_entropy import cross_entropy, linear_cross_entropy
from .model import (BASELINE, ModelConfig, count_params, init_model, model_forward, model_forward_features,
                    output_projection, tree_leaves)

WARMUP_STEPS = int(os.environ.get("NLEARN_WARMUP", "200"))
CHECKPOINT_EVERY = int(os.environ.get("NLEARN_CHECKPOINT_EVERY", "1000"))
PEAK_LR = 1e-3
WEIGHT_DECAY = float(os.environ.get("NLEARN_WD", "0.1"))
BATCH_SIZE = 32


# ---------------------------------------------------------------------------
# loss
# ---------------------------------------------------------------------------


# NLEARN_FUSED_LMHEAD=1 fuses the LM head and the CE (linear_cross_entropy) so
# that the (bs*seq, vocab) logits are never materialised (train.py:24-28).
FUSED_LMHEAD = os.environ.get("NLEARN_FUSED_LMHEAD") == "1"


def batch_loss(params, batch: torch.Tensor, cfg: ModelConfig = BASELINE, fused_lmhead: bool | None = None) -> torch.Tensor:
    """Mean CE of predicting batch[:, 1:] from batch[:, :-1] (train.py:270-299).

    Default: the logits are only read by the CE, so its single pass writes
    dlogits over them (inplace=True): the (bs*seq, vocab) gradient costs no
    extra memory. ``fused_lmhead`` (default: NLEARN_FUSED_LMHEAD) takes the
    linear_cross_entropy path instead (train.py:279-283), which keeps no logits
    between the forward and the backward and recomputes them in the backward.
    """
    # both shifted views in one contiguous copy (one kernel; the lookup and the
    # CE then read them in place)
    input_ids, target_ids = torch.stack((batch[:, :-1], batch[:, 1:])).unbind(0)
    if FUSED_LMHEAD if fused_lmhead is None else fused_lmhead:
        x = model_forward_features(params, input_ids, cfg)
        return linear_cross_entropy(x.reshape(-1, cfg.d_model), output_projection(params), target_ids.reshape(-1))
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


def _rows_ld(t: torch.Tensor):
    """(rows, row stride) of a leaf as the kernels address it: a 2-D tensor with
    unit column stride is rows x stride(0) dense over its storage (padding
    included); anything else is one dense row."""
    if t.dim() == 2 and t.stride(1) == 1 and t.shape[0] > 1:
        return t.shape[0], t.stride(0)
    return 1, t.numel()


def _zeros_with_layout(p: torch.Tensor) -> torch.Tensor:
    """fp32 zeros with p's row layout (a padded matrix stays padded)."""
    rows, ld = _rows_ld(p)
    base = torch.zeros(rows * ld, dtype=torch.float32, device=p.device)
    if p.dim() == 2 and ld != p.shape[1]:
        return base.view(rows, ld)[:, :p.shape[1]]
    return base.view(p.shape)


def attach_grad_buffers(params) -> torch.Tensor:
    """Give every leaf a ``main_grad``: a view into ONE zeroed fp32 buffer, laid
    out like the leaf (64-element aligned starts). The model's backward writes
    each weight gradient straight into it, at the same address every step."""
    leaves = tree_leaves(params)
    sizes = []
    for p in leaves:
        rows, ld = _rows_ld(p)
        sizes.append((rows * ld + 63) // 64 * 64)
    flat = torch.zeros(sum(sizes), dtype=torch.float32, device=leaves[0].device)
    off = 0
    for p, n in zip(leaves, sizes):
        rows, ld = _rows_ld(p)
        seg = flat[off:off + rows * ld]
        if p.dim() == 2 and ld != p.shape[1]:
            p.main_grad = seg.view(rows, ld)[:, :p.shape[1]]
        else:
            p.main_grad = seg.view(p.shape)
        off += n
    return flat


class AdamW:
    """optax.adamw(learning_rate=schedule, b1=.9, b2=.999, eps=1e-8, weight_decay)
    with decoupled decay on every parameter. The schedule is evaluated at the
    update count before the update (optax's ``count``), bias corrections use the
    count after it.

    ``init`` attaches fixed gradient buffers to the leaves (``main_grad``); the
    update is then ONE multi-tensor launch that reads lr and the bias
    corrections from device memory (``state["hyper"]``), so it can live inside
    a captured HIP graph. ``prepare`` writes those scalars for the coming
    update, ``apply`` launches it, ``update`` does both and counts the step.
    Leaves without a buffer fall back to one launch per leaf on ``.grad``."""

    def __init__(self, learning_rate, weight_decay: float = WEIGHT_DECAY, b1: float = 0.9, b2: float = 0.999,
                 eps: float = 1e-8, grad_buffers: bool = True):
        self.lr = learning_rate if callable(learning_rate) else (lambda _c, v=learning_rate: v)
        self.wd, self.b1, self.b2, self.eps = weight_decay, b1, b2, eps
        self.grad_buffers = grad_buffers

    def init(self, params) -> dict:
        leaves = tree_leaves(params)
        flat = attach_grad_buffers(params) if self.grad_buffers else None
        return {"count": 0,
                "mu": [_zeros_with_layout(p) for p in leaves],
                "nu": [_zeros_with_layout(p) for p in leaves],
                "grad_flat": flat,
                "hyper": torch.ones(3, dtype=torch.float32, device=leaves[0].device),
                "table": None}

    def hyper_values(self, count: int):
        t = count + 1
        return float(self.lr(count)), 1.0 - self.b1 ** t, 1.0 - self.b2 ** t

    def prepare(self, state: dict) -> None:
        """Write {lr, bc1, bc2} of update ``state["count"] + 1`` to the device
        (an async copy from freshly pinned memory, ordered on the stream)."""
        h = torch.tensor(self.hyper_values(state["count"]), dtype=torch.float32).pin_memory()
        state["hyper"].copy_(h, non_blocking=True)

    def _table(self, params, state):
        """Device table of the multi-tensor update, rebuilt when a bf16 shadow changed."""
        leaves = tree_leaves(params)
        shadows = []
        for p in leaves:
            sh = getattr(p, "_nl_bf16", None)
            shadows.append(sh if sh is not None and getattr(p, "_nl_bf16_version", None) == p._version else None)
        key = tuple(sh.data_ptr() if sh is not None else 0 for sh in shadows)
        cached = state["table"]
        if cached is not None and cached[0] == key:
            return cached
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("AdamW: parameter layout changed during graph capture")
        T = (_lib.AdamWTensor * len(leaves))()
        for i, (p, m, v, sh) in enumerate(zip(leaves, state["mu"], state["nu"], shadows)):
            rows, ld = _rows_ld(p)
            g = p.main_grad
            if _rows_ld(g) != (rows, ld) or _rows_ld(m) != (rows, ld):
                raise RuntimeError("AdamW: gradient / moment layout differs from the parameter's")
            T[i].p, T[i].g, T[i].m, T[i].v = p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr()
            T[i].rows, T[i].cols = rows, ld
            if sh is not None:
                T[i].shadow, T[i].ld_shadow = sh.data_ptr(), _rows_ld(sh)[1]
        n_chunks = int(_lib.load().nl_adamw_multi_prepare(len(leaves), T))
        if n_chunks < 0:
            raise _lib.NlError("nl_adamw_multi_prepare", -n_chunks, _lib.load().nl_last_error().decode())
        dev_table = torch.frombuffer(bytearray(T), dtype=torch.uint8).to(leaves[0].device)
        state["table"] = (key, dev_table, len(leaves), n_chunks)
        return state["table"]

    def apply(self, params, state: dict) -> None:
        """Launch the update with the scalars already on the device (no host sync)."""
        wgrad.join()  # gradients forked onto the weight-gradient stream must be complete
        leaves = tree_leaves(params)
        stream = torch.cuda.current_stream(leaves[0].device).cuda_stream
        if all(getattr(p, "main_grad", None) is not None for p in leaves):
            _, table, n, n_chunks = self._table(params, state)
            _lib.call("nl_adamw_multi", stream, n, table.data_ptr(), n_chunks, state["hyper"].data_ptr(),
                      self.b1, self.b2, self.eps, self.wd)
            return
        lr, bc1, bc2 = self.hyper_values(state["count"])
        for p, m, v in zip(leaves, state["mu"], state["nu"]):
            g = getattr(p, "main_grad", None)
            g = p.grad if g is None else g
            if g is None:
                continue
            if g.stride() != p.stride():
                g2 = _zeros_with_layout(p)
                g2.copy_(g)
                g = g2
            rows, ld = _rows_ld(p)
            shadow = getattr(p, "_nl_bf16", None)
            sb, ldb = (None, 0)
            if shadow is not None and getattr(p, "_nl_bf16_version", None) == p._version:
                sb, ldb = shadow.data_ptr(), _rows_ld(shadow)[1]
            _lib.call("nl_adamw_step", stream, rows, ld, p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(),
                      sb, ldb, lr, self.b1, self.b2, self.eps, self.wd, bc1, bc2)

    def update(self, params, state: dict) -> dict:
        """Apply one step in place (gradients from ``main_grad`` or ``.grad``)."""
        self.prepare(state)
        self.apply(params, state)
        state["count"] += 1
        return state


def make_train_step(optimizer: AdamW, cfg: ModelConfig = BASELINE, graph: bool = False, warmup: int = 2,
                    overlap_wgrad: bool = True, fused_lmhead: bool | None = None):
    """train_step(params, opt_state, batch) -> (params, opt_state, loss).

    Parameters are updated in place; the loss is a 0-d device tensor (no host
    sync inside the step, as with the jitted step of train.py:328-341).

    graph=True: after ``warmup`` eager steps the whole step (forward, backward,
    AdamW) is captured once into a HIP graph and replayed; the batch is copied
    into the graph's input buffer and lr / bias corrections are written to the
    device before each replay.

    overlap_wgrad: run the weight-gradient kernels on a second stream beside
    the input-gradient chain (kernels.wgrad); results are identical.

    fused_lmhead: the loss through linear_cross_entropy (see ``batch_loss``).
    """
    overlap = wgrad.overlap_weight_grads if overlap_wgrad else _no_overlap

    def eager_step(params, opt_state, batch):
        for p in tree_leaves(params):
            p.grad = None
        loss = batch_loss(params, batch, cfg, fused_lmhead)
        # weight gradients run on a second stream beside the dX chain; the
        # contexts join it and finish the LayerNorm parameter sums before the
        # optimizer reads the gradient buffers
        with overlap(loss.device), fused.defer_layer_norm_param_sums():
            loss.backward()
        with torch.no_grad():
            opt_state = optimizer.update(params, opt_state)
        return params, opt_state, loss.detach()

    if not graph:
        return eager_step
    return _GraphedStep(optimizer, cfg, eager_step, warmup, overlap, fused_lmhead)


@contextlib.contextmanager
def _no_overlap(device=None):
    yield


class _GraphedStep:
    def __init__(self, optimizer, cfg, eager_step, warmup, overlap, fused_lmhead):
        self.opt, self.cfg, self.eager_step, self.warmup = optimizer, cfg, eager_step, warmup
        self.overlap = overlap
        self.fused_lmhead = fused_lmhead
        self.done = 0
        self.graph = None
        self.static_batch = None
        self.static_loss = None
        self.seed = None

    def _capture(self, params, state, batch):
        leaves = tree_leaves(params)
        if not all(getattr(p, "main_grad", None) is not None for p in leaves):
            raise RuntimeError("graph capture needs the optimizer's gradient buffers (AdamW(grad_buffers=True))")
        self.static_batch = batch.detach().clone()
        for p in leaves:
            p.grad = None
        wgrad.prepare(batch.device)  # create the side stream outside the capture
        # the backward's seed d(loss)/d(loss) = 1, made once and kept (every
        # replay reads it): backward() without it records a fill kernel
        self.seed = seed = torch.ones((), dtype=torch.float32, device=batch.device)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            loss = batch_loss(params, self.static_batch, self.cfg, self.fused_lmhead)
            with self.overlap(loss.device), fused.defer_layer_norm_param_sums():
                loss.backward(seed)
            with torch.no_grad():
                self.opt.apply(params, state)
        self.static_loss = loss.detach()
        self.graph = g

    def __call__(self, params, state, batch):
        if self.graph is None:
            if self.done < self.warmup:
                self.done += 1
                return self.eager_step(params, state, batch)
            self._capture(params, state, batch)
        self.static_batch.copy_(batch, non_blocking=True)
        self.opt.prepare(state)
        self.graph.replay()
        state["count"] += 1
        return params, state, self.static_loss.clone()


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
          peak_lr: float = PEAK_LR, log_every: int = 10, cfg: ModelConfig | None = None, run_name=None,
          resume: bool = False, checkpoint_every: int = CHECKPOINT_EVERY) -> list:
    """Offline training loop; returns the per-step losses of the steps it ran.

    As the reference's loop (train.py:537-605): every ``checkpoint_every``
    steps it saves the parameters and the full resume state; ``resume=True``
    continues from ``resume.pkl`` of ``run_name`` when one exists (parameters,
    optimizer state incl. the schedule position, next step)."""
    cfg = cfg or ModelConfig(max_seq_len=max(seq_len, BASELINE.max_seq_len))
    warmup = min(WARMUP_STEPS, max(1, steps) // 5)
    sched = warmup_cosine_decay_schedule(0.0, peak_lr, warmup, max(1, steps), peak_lr / 10)
    opt = AdamW(sched)
    start = 0
    resumed = load_resume_state(opt, run_name) if resume else None
    if resumed is not None:
        params, state, start = resumed
        print(f"Resumed from step {start} (resume.pkl)")
    else:
        params = init_model(seed, cfg)
        state = opt.init(params)
    print(f"params: {count_params(params) / 1e6:.1f} M  bs={batch_size} seq={seq_len} warmup={warmup}")
    step_fn = make_train_step(opt, cfg)
    data = SyntheticTokens(batch_size, seq_len, cfg.vocab_size, seed + start)
    losses = []
    t0 = time.time()
    for step in range(start, steps):
        params, state, loss = step_fn(params, state, data.get_batch())
        losses.append(loss)
        if (step + 1) % log_every == 0 or step + 1 == steps:
            torch.cuda.synchronize()
            dt = time.time() - t0
            print(f"step {step + 1:5d}  loss {loss.item():.4f}  {(step + 1 - start) * batch_size * seq_len / dt:,.0f} tok/s")
        if step > 0 and checkpoint_every > 0 and step % checkpoint_every == 0:
            save_checkpoint(params, step, run_name=run_name)
            save_resume_state(params, state, step + 1, run_name=run_name)
    return [float(l) for l in torch.stack(losses).cpu()] if losses else []


def main(argv=None):
    ap = argparse.ArgumentParser(description="offline nlearn training on the HIP kernels")
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--seq-len", type=int, default=512)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--batch-size", type=int, default=BATCH_SIZE)
    ap.add_argument("--peak-lr", type=float, default=PEAK_LR)
    ap.add_argument("--run-name", default=None)
    ap.add_argument("--resume", action="store_true", help="continue from checkpoints/<run-name>/resume.pkl")
    a = ap.parse_args(argv)
    train(a.steps, a.seq_len, a.seed, a.batch_size, a.peak_lr, run_name=a.run_name, resume=a.resume)


if __name__ == "__main__":
    main()
