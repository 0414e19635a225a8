"""nlearn_amd.train — the training step around the HIP kernels (mirrors nlearn/train.py).

* ``batch_loss(params, batch)``      mean next-token CE of a (bs, seq+1) batch
                                     (train.py:270-299, the batched fused-CE path)
* ``warmup_cosine_decay_schedule``   optax's schedule (train.py:487-495)
* ``AdamW``                          optax.adamw semantics (train.py:504-505) on the
                                     fused HIP kernel; writes the bf16 weight shadows;
                                     ``clip_norm`` chains optax.clip_by_global_norm
                                     in front (NLEARN_GRAD_CLIP, train.py:502-506)
* ``MultiSteps``                     optax.MultiSteps gradient accumulation
                                     (NLEARN_GRAD_ACCUM, train.py:319-325,507-508)
* ``make_train_step(optimizer)``     value_and_grad + update (train.py:328-341), with
                                     the static loss scale (NLEARN_LOSS_SCALE,
                                     train.py:313-316,332-337)
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
import signal
import sys
import threading
import time

import torch

from . import _lib
from .checkpoint import load_checkpoint, load_resume_state, save_checkpoint, save_resume_state  # noqa: F401
from .kernels import fused, wgrad
from .kernels.cross_entropy import cross_entropy, linear_cross_entropy, lm_head_cross_entropy  # noqa: F401
from .model import (BASELINE, ModelConfig, count_params, init_model, model_forward, model_forward_features,
                    output_projection, tree_leaves)

WARMUP_STEPS = int(os.environ.get("NLEARN_WARMUP", "200"))
CHECKPOINT_EVERY = int(os.environ.get("NLEARN_CHECKPOINT_EVERY", "1000"))
PEAK_LR = 1e-3
WEIGHT_DECAY = float(os.environ.get("NLEARN_WD", "0.1"))
BATCH_SIZE = 32
# train.py:313-325,502: static loss scale (1 = off), micro-batches per update,
# global-norm clipping threshold (0 = off)
LOSS_SCALE = float(os.environ.get("NLEARN_LOSS_SCALE", "1.0"))
GRAD_ACCUM = int(os.environ.get("NLEARN_GRAD_ACCUM", "1"))
GRAD_CLIP = float(os.environ.get("NLEARN_GRAD_CLIP", "0"))


# ---------------------------------------------------------------------------
# loss
# ---------------------------------------------------------------------------


# NLEARN_FUSED_LMHEAD=1 fuses the LM head and the CE (linear_cross_entropy) so
# that the (bs*seq, vocab) logits are never materialised (train.py:24-28).
FUSED_LMHEAD = os.environ.get("NLEARN_FUSED_LMHEAD") == "1"
# row chunks of the LM head + CE on the default path (1: one GEMM, then one CE;
# more: each chunk's CE beside the next chunk's GEMM, identical results). Two
# measured fastest on MI355X at bs32 x seq512 (graph replays, 3 rounds on one
# box: 5.98-6.00 ms with one chunk, 5.91-5.92 with two, 5.96 with four).
LMHEAD_CHUNKS = int(os.environ.get("NLEARN_LMHEAD_CHUNKS", "2"))


def batch_loss(params, batch: torch.Tensor, cfg: ModelConfig = BASELINE, fused_lmhead: bool | None = None,
               overlap: bool = True) -> torch.Tensor:
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
    # logits = x . W_lm and the single-pass CE (dlogits over the logits), in
    # LMHEAD_CHUNKS row chunks (each chunk's CE beside the next chunk's GEMM
    # when ``overlap``); the same values as
    # cross_entropy(model_forward(...), targets, inplace=True)
    x = model_forward_features(params, input_ids, cfg)
    return lm_head_cross_entropy(x, output_projection(params), target_ids, LMHEAD_CHUNKS, overlap)


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


def _pinned_to(dst: torch.Tensor, values) -> None:
    """Stream-ordered copy of host scalars into a device tensor (freshly pinned
    memory, so an earlier copy still in flight is never overwritten)."""
    dst.copy_(torch.tensor(values, dtype=torch.float32).pin_memory(), non_blocking=True)


def _same_layout_view(flat: torch.Tensor, like: torch.Tensor, like_flat: torch.Tensor) -> torch.Tensor:
    """The view of ``flat`` at the position and with the strides ``like`` has in ``like_flat``."""
    return torch.as_strided(flat, like.shape, like.stride(), like.storage_offset() - like_flat.storage_offset())


class AdamW:
    """optax.adamw(learning_rate=schedule, b1=.9, b2=.999, eps=1e-8, weight_decay)
    with decoupled decay on every parameter. The schedule is evaluated at the
    update count before the update (optax's ``count``), bias corrections use the
    count after it. ``clip_norm`` > 0 puts optax.clip_by_global_norm(clip_norm)
    in front (train.py:502-506): the global norm is computed on the device and
    read there by the update, so no host synchronisation is involved.

    ``init`` attaches fixed gradient buffers to the leaves (``main_grad``); the
    update is then ONE multi-tensor launch that reads lr and the bias
    corrections from device memory (``state["hyper"]``), so it can live inside
    a captured HIP graph. The step protocol, shared with ``MultiSteps``:
    ``prepare`` writes the device scalars for the coming step, ``apply`` launches
    the capturable work, ``finish`` runs what follows it outside a graph (nothing
    here), ``advance`` counts the step; ``update`` does all four. Leaves without
    a buffer fall back to one launch per leaf on ``.grad`` (no clipping there)."""

    def __init__(self, learning_rate, weight_decay: float = WEIGHT_DECAY, b1: float = 0.9, b2: float = 0.999,
                 eps: float = 1e-8, grad_buffers: bool = True, clip_norm: float = 0.0):
        self.lr = learning_rate if callable(learning_rate) else (lambda _c, v=learning_rate: v)
        self.wd, self.b1, self.b2, self.eps = weight_decay, b1, b2, eps
        self.grad_buffers = grad_buffers
        self.clip_norm = float(clip_norm)

    def init(self, params) -> dict:
        leaves = tree_leaves(params)
        dev = leaves[0].device
        flat = attach_grad_buffers(params) if self.grad_buffers else None
        state = {"count": 0,
                 "mu": [_zeros_with_layout(p) for p in leaves],
                 "nu": [_zeros_with_layout(p) for p in leaves],
                 "grad_flat": flat,
                 # the gradients the update reads: main_grad (None) or views of grad_src_flat
                 "grads": None, "grad_src_flat": flat,
                 "hyper": torch.ones(3, dtype=torch.float32, device=dev),
                 "unscale": torch.ones(2, dtype=torch.float32, device=dev), "unscale_value": 1.0,
                 "table": None}
        if self.clip_norm > 0 and flat is not None:
            state["gnorm"] = torch.zeros(1, dtype=torch.float32, device=dev)
            n = flat.numel()
            state["norm_ws"] = torch.empty(max(int(_lib.load().nl_global_norm_ws_bytes(n)), 16) // 4,
                                           dtype=torch.float32, device=dev)
        return state

    def hyper_values(self, count: int):
        t = count + 1
        return float(self.lr(count)), 1.0 - self.b1 ** t, 1.0 - self.b2 ** t

    def prepare(self, state: dict, loss_scale: float = 1.0) -> None:
        """Write {lr, bc1, bc2} of update ``state["count"] + 1`` to the device
        (and the loss-scale divisor, when it changed)."""
        _pinned_to(state["hyper"], self.hyper_values(state["count"]))
        if loss_scale != state["unscale_value"]:
            _pinned_to(state["unscale"], (float(loss_scale), 1.0))
            state["unscale_value"] = float(loss_scale)

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
        grads = state["grads"] or [p.main_grad for p in leaves]
        T = (_lib.AdamWTensor * len(leaves))()
        for i, (p, g, m, v, sh) in enumerate(zip(leaves, grads, state["mu"], state["nu"], shadows)):
            rows, ld = _rows_ld(p)
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

    def apply(self, params, state: dict, loss_scale: float = 1.0) -> None:
        """Launch the update with the scalars already on the device (no host sync):
        gradients / loss_scale (in place), the global norm if clipping, AdamW."""
        wgrad.join()  # gradients forked onto the weight-gradient stream must be complete
        leaves = tree_leaves(params)
        stream = torch.cuda.current_stream(leaves[0].device).cuda_stream
        if state["grads"] is not None or all(getattr(p, "main_grad", None) is not None for p in leaves):
            src = state["grad_src_flat"]
            if loss_scale != 1.0:
                # train.py:335-336 divides the gradients by the loss scale before the update
                _lib.call("nl_grad_accumulate", stream, src.numel(), src.data_ptr(), src.data_ptr(),
                          state["unscale"].data_ptr())
            _, table, n, n_chunks = self._table(params, state)
            if self.clip_norm > 0:
                ws = state["norm_ws"]
                _lib.call("nl_global_norm", stream, src.numel(), src.data_ptr(), state["gnorm"].data_ptr(),
                          ws.data_ptr(), ws.numel() * 4)
                _lib.call("nl_adamw_multi_clip", stream, n, table.data_ptr(), n_chunks, state["hyper"].data_ptr(),
                          self.b1, self.b2, self.eps, self.wd, state["gnorm"].data_ptr(), self.clip_norm)
            else:
                _lib.call("nl_adamw_multi", stream, n, table.data_ptr(), n_chunks, state["hyper"].data_ptr(),
                          self.b1, self.b2, self.eps, self.wd)
            return
        if self.clip_norm > 0 or loss_scale != 1.0:
            raise RuntimeError("AdamW: clipping and loss scaling need the gradient buffers (grad_buffers=True)")
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

    def finish(self, params, state: dict) -> None:
        """Nothing runs after the captured part of an AdamW step."""

    def advance(self, state: dict) -> None:
        state["count"] += 1

    def update(self, params, state: dict, loss_scale: float = 1.0) -> dict:
        """Apply one step in place (gradients from ``main_grad`` or ``.grad``)."""
        self.prepare(state, loss_scale)
        self.apply(params, state, loss_scale)
        self.finish(params, state)
        self.advance(state)
        return state


class MultiSteps:
    """optax.MultiSteps(inner, every_k_schedule=k) (train.py:319-325,507-508).

    Every call is one micro-step. Its gradients (divided by the loss scale)
    join the running mean acc + (g - acc) / (i + 1) of the micro-steps so far
    (optax's formula, one HBM pass: ``nl_grad_accumulate``); every k-th call
    then runs the inner optimizer (clipping and AdamW) on that mean and starts
    over, and the parameters do not change on the other calls. The inner
    count, and with it the schedule, advances once per k micro-steps. The
    per-micro-step work is capturable; the inner update of the k-th call runs
    after the captured part (``finish``), reading the same fixed buffers."""

    def __init__(self, inner: AdamW, every_k: int):
        if every_k < 1:
            raise ValueError("MultiSteps: every_k must be >= 1")
        if not inner.grad_buffers:
            raise ValueError("MultiSteps: the inner optimizer needs gradient buffers")
        self.inner, self.k = inner, int(every_k)

    def init(self, params) -> dict:
        inner = self.inner.init(params)
        flat = inner["grad_flat"]
        acc = torch.zeros_like(flat)
        inner["grads"] = [_same_layout_view(acc, p.main_grad, flat) for p in tree_leaves(params)]
        inner["grad_src_flat"] = acc
        return {"inner": inner, "count": inner["count"], "mini_step": 0, "acc_flat": acc,
                "coef": torch.ones(2, dtype=torch.float32, device=flat.device),
                "mu": inner["mu"], "nu": inner["nu"]}

    def _final(self, state) -> bool:
        return state["mini_step"] + 1 == self.k

    def prepare(self, state: dict, loss_scale: float = 1.0) -> None:
        _pinned_to(state["coef"], (float(loss_scale), float(state["mini_step"] + 1)))
        if self._final(state):
            self.inner.prepare(state["inner"])

    def apply(self, params, state: dict, loss_scale: float = 1.0) -> None:
        wgrad.join()
        stream = torch.cuda.current_stream(state["acc_flat"].device).cuda_stream
        src = state["inner"]["grad_flat"]
        _lib.call("nl_grad_accumulate", stream, src.numel(), state["acc_flat"].data_ptr(), src.data_ptr(),
                  state["coef"].data_ptr())

    def finish(self, params, state: dict) -> None:
        if self._final(state):
            self.inner.apply(params, state["inner"])

    def advance(self, state: dict) -> None:
        if self._final(state):
            self.inner.advance(state["inner"])
            state["mini_step"] = 0
        else:
            state["mini_step"] += 1
        state["count"] = state["inner"]["count"]

    def update(self, params, state: dict, loss_scale: float = 1.0) -> dict:
        self.prepare(state, loss_scale)
        self.apply(params, state, loss_scale)
        self.finish(params, state)
        self.advance(state)
        return state


def make_train_step(optimizer, cfg: ModelConfig = BASELINE, graph: bool = False, warmup: int = 2,
                    overlap_wgrad: bool = True, fused_lmhead: bool | None = None, loss_scale: float | None = None):
    """train_step(params, opt_state, batch) -> (params, opt_state, loss).

    ``optimizer`` is an ``AdamW`` or a ``MultiSteps`` around one (the
    reference's make_train_step takes the optax optimizer the same way,
    train.py:328-341). Parameters are updated in place; the loss is a 0-d
    device tensor (no host sync inside the step, as with the jitted step).

    loss_scale (default NLEARN_LOSS_SCALE): the backward starts from
    d(loss)/d(loss) = loss_scale, so every gradient is scaled by it, and the
    optimizer divides it out before use (train.py:313-316,332-337); the loss
    returned is the unscaled one.

    graph=True: after ``warmup`` eager steps the whole step (forward, backward
    and the optimizer's capturable part) is captured once into a HIP graph
    and replayed; the batch is copied into the graph's input buffer and the
    optimizer's scalars are written to the device before each replay.

    overlap_wgrad: run the weight-gradient kernels on a second stream beside
    the input-gradient chain (kernels.wgrad), and each LM-head chunk's CE
    beside the next chunk's GEMM; results are identical. False runs every
    kernel on the current stream.

    fused_lmhead: the loss through linear_cross_entropy (see ``batch_loss``).
    """
    check_hw_queues()
    overlap = wgrad.overlap_weight_grads if overlap_wgrad else _no_overlap
    scale = LOSS_SCALE if loss_scale is None else float(loss_scale)
    if not scale > 0:
        raise ValueError("make_train_step: loss_scale must be > 0")

    def eager_step(params, opt_state, batch):
        for p in tree_leaves(params):
            p.grad = None
        loss = batch_loss(params, batch, cfg, fused_lmhead, overlap_wgrad)
        seed = None if scale == 1.0 else torch.full((), scale, dtype=torch.float32, device=loss.device)
        # weight gradients run on a second stream beside the dX chain; the
        # contexts join it and finish the LayerNorm parameter sums before the
        # optimizer reads the gradient buffers
        with overlap(loss.device), fused.defer_layer_norm_param_sums():
            loss.backward(seed)
        with torch.no_grad():
            opt_state = optimizer.update(params, opt_state, scale)
        return params, opt_state, loss.detach()

    if not graph:
        return eager_step
    return _GraphedStep(optimizer, cfg, eager_step, warmup, overlap, fused_lmhead, scale)


@contextlib.contextmanager
def _no_overlap(device=None):
    yield


# The fewest hardware queues per device the training step has run with. The
# HIP runtime maps streams onto GPU_MAX_HW_QUEUES queues (default 4); the step
# uses up to three streams of its own (the current one, the weight-gradient
# stream, the op-internal side stream) plus graph capture's. It has run with
# 4, 8 and 16 queues. A process with GPU_MAX_HW_QUEUES=2 ended in a host
# segmentation fault before its first timed step, with no error from any HIP
# call; the cause was not found, so fewer queues than 4 are refused.
MIN_HW_QUEUES = 4


def check_hw_queues(env=None) -> None:
    """Raise if GPU_MAX_HW_QUEUES asks for fewer hardware queues than the step
    has been run with (see MIN_HW_QUEUES); unset or unparsable values leave the
    runtime's default of 4."""
    raw = (os.environ if env is None else env).get("GPU_MAX_HW_QUEUES")
    try:
        n = int(raw) if raw is not None else None
    except ValueError:
        n = None
    if n is not None and 0 < n < MIN_HW_QUEUES:
        raise RuntimeError(
            f"GPU_MAX_HW_QUEUES={n}: the training step has only been run with {MIN_HW_QUEUES} or more hardware "
            f"queues per device (a run with 2 ended in a segmentation fault whose cause is not known); "
            f"unset it or set it to at least {MIN_HW_QUEUES}")


class _GraphedStep:
    def __init__(self, optimizer, cfg, eager_step, warmup, overlap, fused_lmhead, loss_scale):
        self.opt, self.cfg, self.eager_step, self.warmup = optimizer, cfg, eager_step, warmup
        self.overlap = overlap
        self.fused_lmhead = fused_lmhead
        self.loss_scale = loss_scale
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
        # the backward's seed d(loss)/d(loss) (the loss scale), made once and
        # kept (every replay reads it): backward() without it records a fill kernel
        self.seed = seed = torch.full((), self.loss_scale, dtype=torch.float32, device=batch.device)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            loss = batch_loss(params, self.static_batch, self.cfg, self.fused_lmhead, self.overlap is not _no_overlap)
            with self.overlap(loss.device), fused.defer_layer_norm_param_sums():
                loss.backward(seed)
            with torch.no_grad():
                self.opt.apply(params, state, self.loss_scale)
        self.static_loss = loss.detach()
        self.graph = g

    def __call__(self, params, state, batch):
        if self.graph is None:
            if self.done < self.warmup:
                self.done += 1
                return self.eager_step(params, state, batch)
            self._capture(params, state, batch)
        self.static_batch.copy_(batch, non_blocking=True)
        self.opt.prepare(state, self.loss_scale)
        self.graph.replay()
        with torch.no_grad():
            self.opt.finish(params, state)
        self.opt.advance(state)
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


class GracefulStop:
    """SIGINT / SIGTERM set a flag instead of ending the process; the loop
    checks it after each step (train.py:556-562). Installed only from the main
    thread (Python delivers signals there); the previous handlers come back on
    exit."""

    SIGNALS = (signal.SIGINT, signal.SIGTERM)

    def __init__(self):
        self.requested = False
        self._old = {}

    def _handle(self, signum, frame):
        print("\nInterrupt received — will save checkpoint and exit after this step.", flush=True)
        self.requested = True

    def __enter__(self):
        if threading.current_thread() is threading.main_thread():
            for sig in self.SIGNALS:
                self._old[sig] = signal.signal(sig, self._handle)
        return self

    def __exit__(self, *exc):
        for sig, old in self._old.items():
            signal.signal(sig, old)
        self._old.clear()
        return False


def train(steps: int = 20, seq_len: int = 512, seed: int = 0, batch_size: int = BATCH_SIZE,
          peak_lr: float = PEAK_LR, log_every: int = 10, cfg: ModelConfig | None = None, run_name=None,
          resume: bool = False, checkpoint_every: int = CHECKPOINT_EVERY) -> list:
    """Offline training loop; returns the per-step losses of the steps it ran.

    As the reference's loop (train.py:537-622): every ``checkpoint_every``
    steps it saves the parameters and the full resume state; ``resume=True``
    continues from ``resume.pkl`` of ``run_name`` when one exists (parameters,
    optimizer state incl. the schedule position, next step). SIGINT or SIGTERM
    finishes the current step, saves the parameters (``step_NNNNNN.pkl`` of
    that step) and the resume state, and exits the process with status 0
    (train.py:556-562,604-609). The last step's parameters are saved as
    ``step_<steps>.pkl`` (train.py:612)."""
    cfg = cfg or ModelConfig(max_seq_len=max(seq_len, BASELINE.max_seq_len))
    # with GRAD_ACCUM micro-steps per update the schedule advances per
    # effective update (train.py:483-495)
    eff_updates = max(1, steps // GRAD_ACCUM)
    warmup = min(WARMUP_STEPS, eff_updates // 5)
    sched = warmup_cosine_decay_schedule(0.0, peak_lr, warmup, eff_updates, peak_lr / 10)
    opt = AdamW(sched, clip_norm=GRAD_CLIP)
    if GRAD_ACCUM > 1:
        opt = MultiSteps(opt, GRAD_ACCUM)
        print(f"Gradient accumulation: {GRAD_ACCUM} micro-batches/update "
              f"(effective batch {batch_size * GRAD_ACCUM}, {eff_updates} updates)")
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
    with GracefulStop() as stop:
        for step in range(start, steps):
            params, state, loss = step_fn(params, state, data.get_batch())
            losses.append(loss)
            if (step + 1) % log_every == 0 or step + 1 == steps:
                torch.cuda.synchronize()
                dt = time.time() - t0
                print(f"step {step + 1:5d}  loss {loss.item():.4f}  "
                      f"{(step + 1 - start) * batch_size * seq_len / dt:,.0f} tok/s", flush=True)
            if step > 0 and checkpoint_every > 0 and step % checkpoint_every == 0:
                save_checkpoint(params, step, run_name=run_name)
                save_resume_state(params, state, step + 1, run_name=run_name)
            if stop.requested:
                print("Saving checkpoint before exit...", flush=True)
                save_checkpoint(params, step, run_name=run_name)
                save_resume_state(params, state, step + 1, run_name=run_name)
                sys.exit(0)
    if steps > start:
        save_checkpoint(params, steps, run_name=run_name)
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
