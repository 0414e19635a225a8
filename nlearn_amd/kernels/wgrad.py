"""nlearn_amd.kernels.wgrad — weight gradients on a second stream.

In a layer's backward pass the weight gradients (X^T dY products, bias
column sums) feed nothing but the optimizer, while the input gradient dX feeds
the next layer's backward. Inside ``overlap_weight_grads()`` the weight-gradient
kernels are forked onto a second HIP stream (default priority) at the point
their inputs are ready, so they run beside the dX chain instead of between its
steps; the optimizer joins the stream (``join()``) before it reads the
gradient buffers. This is a scheduling change only: every kernel, operand and
summation order is the same as on one stream.

Rules that keep this safe under the caching allocator and HIP graph capture:

* the forked work allocates nothing: workspaces are allocated on the current
  stream before the fork and handed in;
* every tensor the forked work reads or writes stays referenced until
  ``join()``, so its memory cannot be reused while the side stream may still
  touch it;
* the side stream always waits for the current stream first, and the current
  stream waits for the side stream at ``join()`` (fork and join, as graph
  capture requires).

The autograd engine runs backward functions on its own thread, so the state
is module-global, not thread-local; one overlapped step runs at a time.
"""
from __future__ import annotations

import contextlib

import torch

_side: dict = {}        # (device index, slot) -> stream; slot 0: weight gradients, 1: within one op
_active: dict | None = None


def _side_stream(dev: torch.device, slot: int = 0) -> torch.cuda.Stream:
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    s = _side.get((idx, slot))
    if s is None:
        s = torch.cuda.Stream(device=idx)  # default priority
        _side[(idx, slot)] = s
    return s


def prepare(device=None) -> None:
    """Create the device's side streams now (e.g. before a graph capture)."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    _side_stream(dev, 0)
    _side_stream(dev, 1)


def split(first, second, *keep) -> None:
    """Run ``first()`` on the current stream and ``second()`` (which must not
    allocate) on the op-internal side stream, concurrently when overlapping is
    active, and join before returning: the current stream then waits for
    both. ``keep``: every tensor ``second`` touches (referenced until here)."""
    if _active is None:
        first()
        second()
        return
    main = torch.cuda.current_stream()
    aux = _side_stream(_active["dev"], 1)
    aux.wait_stream(main)
    with torch.cuda.stream(aux):
        second()
    first()
    main.wait_stream(aux)
    del keep


def active() -> bool:
    return _active is not None


@contextlib.contextmanager
def overlap_weight_grads(device=None):
    """Within the block, ``fork()`` runs weight-gradient work on a side stream;
    the block joins that stream on exit (and ``join()`` may join earlier)."""
    global _active
    if _active is not None:
        raise RuntimeError("overlap_weight_grads() does not nest")
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    _active = {"side": _side_stream(dev), "keep": [], "main": torch.cuda.current_stream(dev), "forked": False,
               "dev": dev}
    try:
        yield
    finally:
        try:
            join()
        finally:
            _active = None


def fork(fn, *keep):
    """Run ``fn()`` (which must not allocate) after all work queued so far on
    the current stream, on the side stream when overlapping is active, else
    inline. ``keep``: every tensor ``fn`` touches."""
    if _active is None:
        return fn()
    main = torch.cuda.current_stream()
    side = _active["side"]
    side.wait_stream(main)
    _active["keep"].extend(keep)
    _active["forked"] = True
    with torch.cuda.stream(side):
        return fn()


def join() -> None:
    """Make the stream that opened ``overlap_weight_grads()`` wait for all
    forked work; releases the tensors kept for it."""
    if _active is None or not _active["forked"]:
        return
    _active["main"].wait_stream(_active["side"])
    _active["keep"].clear()
    _active["forked"] = False
