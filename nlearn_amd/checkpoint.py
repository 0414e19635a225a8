"""nlearn_amd.checkpoint — the reference's checkpoint files (train.py:36-99).

* ``save_checkpoint(params, step, run_name)`` writes
  ``checkpoints[/run_name]/step_NNNNNN.pkl``: a pickle of the parameter tree as
  nested dicts / lists of float32 NumPy arrays, the layout ``jax.device_get``
  gives the reference (train.py:45-59).
* ``load_checkpoint(path)`` reads one back as that NumPy tree; with ``device``
  it returns device parameters ready for the training step (train.py:62-68).
* ``save_resume_state`` / ``load_resume_state``: parameters, optimizer state
  and the next step in ``resume.pkl``, written to a temporary file and renamed
  so that a crash mid-write leaves the previous file intact (train.py:71-99).
  The optimizer state is this package's AdamW state (update count and the
  two moment trees); the reference pickles optax's state objects instead,
  which only optax can rebuild, so a reference ``resume.pkl`` is not read.

Loading never runs code from the file: the unpickler resolves only NumPy's
array constructors and dtype, so a file holding anything else is refused.
"""
from __future__ import annotations

import io
import os
import pickle

import numpy as np

CHECKPOINT_DIR = "checkpoints"

# the only globals a parameter pickle needs (NumPy 1.x and 2.x module names)
_ALLOWED = {
    ("numpy", "ndarray"),
    ("numpy", "dtype"),
    ("numpy.core.multiarray", "_reconstruct"),
    ("numpy.core.multiarray", "scalar"),
    ("numpy._core.multiarray", "_reconstruct"),
    ("numpy._core.multiarray", "scalar"),
    ("numpy.core.numeric", "_frombuffer"),      # protocol 5: array from its raw bytes
    ("numpy._core.numeric", "_frombuffer"),
}


class _ArrayUnpickler(pickle.Unpickler):
    def find_class(self, module, name):
        if (module, name) in _ALLOWED:
            return super().find_class(module, name)
        raise pickle.UnpicklingError(f"checkpoint: refusing to load {module}.{name} (only NumPy arrays are allowed)")


def _load(path: str):
    with open(path, "rb") as f:
        return _ArrayUnpickler(io.BytesIO(f.read())).load()


def to_numpy(tree):
    """Device (or host) tensors -> the same tree of float32 NumPy arrays."""
    import torch

    if isinstance(tree, dict):
        return {k: to_numpy(v) for k, v in tree.items()}
    if isinstance(tree, (list, tuple)):
        return [to_numpy(v) for v in tree]
    if isinstance(tree, torch.Tensor):
        return tree.detach().to("cpu", torch.float32).contiguous().numpy().copy()
    return np.asarray(tree)


def to_device(tree, device="cuda"):
    """NumPy parameter tree -> device parameters (fp32 leaves with gradients,
    the padded row stride of model.device_param)."""
    from .model import device_param, tree_map

    return tree_map(lambda a: device_param(np.asarray(a, np.float32), device), tree)


def _dir(run_name):
    return os.path.join(CHECKPOINT_DIR, run_name) if run_name else CHECKPOINT_DIR


def _atomic_dump(obj, path: str) -> None:
    os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        pickle.dump(obj, f, protocol=pickle.HIGHEST_PROTOCOL)
    os.replace(tmp, path)


def save_checkpoint(params, step: int, run_name=None) -> str:
    """Save the parameters at ``step`` (train.py:45-59); returns the path."""
    path = os.path.join(_dir(run_name), f"step_{step:06d}.pkl")
    _atomic_dump(to_numpy(params), path)
    print(f"  Checkpoint saved: {path}")
    return path


def load_checkpoint(path: str, device=None):
    """The parameter tree saved by ``save_checkpoint`` (train.py:62-68): NumPy
    arrays, or device parameters when ``device`` is given."""
    tree = _load(path)
    return to_device(tree, device) if device is not None else tree


def _resume_path(run_name) -> str:
    return os.path.join(_dir(run_name), "resume.pkl")


def save_resume_state(params, opt_state: dict, step: int, run_name=None) -> str:
    """Parameters, AdamW state and the next step, atomically (train.py:76-89)."""
    so = {"count": int(opt_state["count"]), "mu": to_numpy(opt_state["mu"]), "nu": to_numpy(opt_state["nu"])}
    if "mini_step" in opt_state:  # MultiSteps: the micro-step and the running mean so far
        so["mini_step"] = int(opt_state["mini_step"])
        so["acc"] = to_numpy(opt_state["acc_flat"])
    state = {"params": to_numpy(params), "opt_state": so, "step": int(step)}
    path = _resume_path(run_name)
    _atomic_dump(state, path)
    return path


def load_resume_state(optimizer, run_name=None, device="cuda"):
    """(params, opt_state, next_step) from ``resume.pkl``, or None without one
    (train.py:92-99). ``optimizer.init`` builds the state around the restored
    parameters (gradient buffers, tables); the moments and the update count
    are then those saved."""
    import torch

    path = _resume_path(run_name)
    if not os.path.exists(path):
        return None
    saved = _load(path)
    params = to_device(saved["params"], device)
    state = optimizer.init(params)
    so = saved["opt_state"]
    if len(so["mu"]) != len(state["mu"]) or len(so["nu"]) != len(state["nu"]):
        raise ValueError("resume: the optimizer state does not match the parameter tree")
    with torch.no_grad():
        for dst, src in zip(state["mu"] + state["nu"], list(so["mu"]) + list(so["nu"])):
            if tuple(dst.shape) != tuple(np.shape(src)):
                raise ValueError(f"resume: moment shape {np.shape(src)} != {tuple(dst.shape)}")
            dst.copy_(torch.from_numpy(np.asarray(src, np.float32)))
    state["count"] = int(so["count"])
    if "inner" in state:  # MultiSteps around AdamW
        state["inner"]["count"] = int(so["count"])
        if "mini_step" in so:
            acc = np.asarray(so["acc"], np.float32)
            if acc.shape != tuple(state["acc_flat"].shape):
                raise ValueError("resume: the accumulated gradient does not match the parameter tree")
            state["mini_step"] = int(so["mini_step"])
            with torch.no_grad():
                state["acc_flat"].copy_(torch.from_numpy(acc))
    return params, state, int(saved["step"])
