"""ctypes binding of ``libnlearn_hip.so`` (the C ABI in include/nlearn_hip.h).

There is no fallback: if the library is missing or a call fails, an exception
is raised. Device buffers come from torch (HIP) tensors; this module only
passes their addresses and the current HIP stream.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("NLEARN_HIP_LIB", Path(__file__).resolve().parent / "libnlearn_hip.so"))

NL_OK, NL_EINVAL, NL_EALIGN, NL_EUNSUPPORTED, NL_ELAUNCH = 0, 1, 2, 3, 4
NL_OP_N, NL_OP_T = 0, 1
NL_DTYPE_F32, NL_DTYPE_BF16 = 0, 1


class AttnStride(ctypes.Structure):
    """``nl_attn_stride``: element strides of (batch, head, row); d is contiguous."""

    _fields_ = [("batch", ctypes.c_int64), ("head", ctypes.c_int64), ("row", ctypes.c_int64)]


class AdamWTensor(ctypes.Structure):
    """``nl_adamw_tensor``: one leaf of the multi-tensor AdamW table."""

    _fields_ = [("p", ctypes.c_void_p), ("g", ctypes.c_void_p), ("m", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("shadow", ctypes.c_void_p), ("ld_shadow", ctypes.c_int64), ("rows", ctypes.c_int64),
                ("cols", ctypes.c_int64), ("chunk0", ctypes.c_int64)]


class NlError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_D = ctypes.c_double
_S = AttnStride

# name -> argtypes (restype is int unless listed in _RESTYPES)
_SIGNATURES = {
    "nl_strerror": [_I],
    "nl_last_error": [],
    "nl_version": [],
    "nl_gemm": [_P, _I, _I, _I, _I, _I, _F, _P, _I64, _P, _I64, _F, _P, _I, _I64, _P],
    "nl_gemm_ws_bytes": [_I, _I, _I, _I, _I],
    "nl_gemm_ex": [_P, _I, _I, _I, _I, _I, _F, _P, _I64, _P, _I64, _F, _P, _I, _I64, _P, _P, ctypes.c_size_t],
    "nl_gemm_fused": [_P, _I, _I, _I, _I, _I, _F, _P, _I64, _P, _I64, _F, _P, _I, _I64, _P, _I, _P, _P, _I64, _P,
                      ctypes.c_size_t],
    "nl_flash_attention_fwd": [_P, _I, _I, _I, _I, _F, _I, _P, _S, _P, _S, _P, _S, _P, _S, _P],
    "nl_flash_attention_bwd_preprocess": [_P, _I, _I, _I, _I, _P, _S, _P, _S, _P],
    "nl_flash_attention_bwd_dq": [_P, _I, _I, _I, _I, _F, _I, _P, _S, _P, _S, _P, _S, _P, _S, _P, _P, _P, _S],
    "nl_flash_attention_bwd_dkdv": [_P, _I, _I, _I, _I, _F, _I, _P, _S, _P, _S, _P, _S, _P, _S, _P, _P,
                                    _P, _S, _P, _S],
    "nl_flash_attention_bwd_ws_bytes": [_I, _I, _I],
    "nl_flash_attention_bwd": [_P, _I, _I, _I, _I, _F, _I, _P, _S, _P, _S, _P, _S, _P, _S, _P, _S, _P,
                               _P, _S, _P, _S, _P, _S, _P],
    "nl_flash_attention_bwd_noalloc": [_P, _I, _I, _I, _I, _F, _I, _P, _S, _P, _S, _P, _S, _P, _S, _P, _S, _P,
                                       _P, _S, _P, _S, _P, _S],
    "nl_ce_fwd": [_P, _I, _I, _P, _I64, _P, _P, _P],
    "nl_ce_bwd": [_P, _I, _I, _P, _I64, _P, _P, _F, _P, _I64],
    "nl_ce_fwd_bwd": [_P, _I, _I, _P, _I64, _P, _P, _P, _F, _P, _I64],
    "nl_lce_ws_bytes": [_I, _I],
    "nl_lce_fwd": [_P, _I, _I, _I, _P, _I64, _P, _I64, _P, _P, _P, _P, ctypes.c_size_t],
    "nl_lce_bwd_dlogits": [_P, _I, _I, _I, _I, _I, _P, _I64, _P, _I64, _P, _P, _F, _P, _P, _I64],
    "nl_mean_f32": [_P, _P, _I, _P],
    "nl_scale_bf16_by_device_scalar": [_P, _P, _I64, _I64, _I64, _P],
    "nl_adamw_step": [_P, _I64, _I64, _P, _P, _P, _P, _P, _I64, _F, _D, _D, _F, _F, _F, _F],
    "nl_adamw_multi_prepare": [_I, _P],
    "nl_adamw_multi": [_P, _I, _P, _I64, _P, _D, _D, _F, _F],
    "nl_adamw_multi_clip": [_P, _I, _P, _I64, _P, _D, _D, _F, _F, _P, _F],
    "nl_global_norm_ws_bytes": [_I64],
    "nl_global_norm": [_P, _I64, _P, _P, _P, ctypes.c_size_t],
    "nl_grad_accumulate": [_P, _I64, _P, _P, _P],
    "nl_layernorm_fwd": [_P, _I, _I, _P, _P, _P, _P, _P, _F, _P, _P, _P],
    "nl_layernorm_bwd_ws_bytes": [_I, _I],
    "nl_layernorm_bwd": [_P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, ctypes.c_size_t],
    "nl_layernorm_bwd_deferred": [_P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _I, _I, _P, _P, _P,
                                  _I],
    "nl_layernorm_param_sums": [_P, _I, _I, _P, _P, _P, _I],
    "nl_colsum_ws_bytes": [_I, _I],
    "nl_colsum_bf16": [_P, _I, _I, _P, _I64, _P, _I, _P, ctypes.c_size_t],
    "nl_embedding_fwd": [_P, _I, _I, _I, _I, _P, _P, _P, _P],
    "nl_embedding_bwd_ws_bytes": [_I, _I, _I, _I],
    "nl_embedding_bwd": [_P, _I, _I, _I, _I, _P, _P, _P, _P, _I, _P, ctypes.c_size_t],
}
_RESTYPES = {
    "nl_strerror": ctypes.c_char_p,
    "nl_last_error": ctypes.c_char_p,
    "nl_version": ctypes.c_char_p,
    "nl_flash_attention_bwd_ws_bytes": ctypes.c_size_t,
    "nl_gemm_ws_bytes": ctypes.c_size_t,
    "nl_layernorm_bwd_ws_bytes": ctypes.c_size_t,
    "nl_adamw_multi_prepare": ctypes.c_int64,
    "nl_colsum_ws_bytes": ctypes.c_size_t,
    "nl_lce_ws_bytes": ctypes.c_size_t,
    "nl_global_norm_ws_bytes": ctypes.c_size_t,
    "nl_embedding_bwd_ws_bytes": ctypes.c_size_t,
}

EXPORTED = tuple(_SIGNATURES)

_lib = None


def load() -> ctypes.CDLL:
    """Load the library once (after torch, so both share one HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m nlearn_amd._build` "
            "(there is no non-HIP fallback)")
    try:
        import torch  # noqa: F401  (binds the process to torch's HIP runtime first)
    except ImportError:
        pass
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    _lib = lib
    return lib


_probe = None


def set_probe(probe) -> None:
    """Install (or clear with None) a callable ``probe(name, args) -> ctx``.

    When set, every entry point call runs inside the context manager the probe
    returns (or unwrapped if it returns None); used by bench.py to bracket
    kernels with HIP events on the stream they are launched on."""
    global _probe
    _probe = probe


def call(name: str, *args) -> None:
    """Invoke an ``nl_*`` status-returning entry point; raise NlError on failure."""
    lib = load()
    ctx = _probe(name, args) if _probe is not None else None
    if ctx is None:
        rc = getattr(lib, name)(*args)
    else:
        with ctx:
            rc = getattr(lib, name)(*args)
    if rc != NL_OK:
        msg = lib.nl_last_error().decode() or lib.nl_strerror(rc).decode()
        raise NlError(name, rc, msg)


def ws_bytes(batch: int, heads: int, seq: int) -> int:
    return int(load().nl_flash_attention_bwd_ws_bytes(batch, heads, seq))
