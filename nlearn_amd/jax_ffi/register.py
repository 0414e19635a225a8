"""Register the reference's jax.ffi targets with the handlers of nlearn_jax_ffi.cc.

On a JAX-ROCm install, after building ``libnlearn_jax_ffi.so`` (see the header
of nlearn_jax_ffi.cc), call ``register()`` once at import in nlearn's
``attention.py``, ``kernels/gemm.py`` and ``kernels/cross_entropy.py`` (beside
their ``ffi_call`` sites). JAX is not installed in this repository's image;
nothing here runs in its tests except ``TARGETS`` being checked against the
handler symbols the C++ file defines.
"""
from __future__ import annotations

import ctypes
import os

# (target name used by the reference's ffi_call, handler symbol in nlearn_jax_ffi.cc)
TARGETS = (
    ("flash_attention_fwd", "nl_flash_attention_fwd_ffi"),       # attention.py:82-91
    ("flash_attention_bwd_dq", "nl_flash_attention_bwd_dq_ffi"),  # attention.py:117-121
    ("flash_attention_bwd_dkdv", "nl_flash_attention_bwd_dkdv_ffi"),  # attention.py:122-127
    ("gemm", "nl_gemm_ffi"),                                     # gemm.py:32-40
    ("gemm_nt", "nl_gemm_nt_ffi"),                               # gemm.py:74 without B.T
    ("gemm_tn", "nl_gemm_tn_ffi"),                               # gemm.py:75 without A.T
    ("ce_fwd", "nl_ce_fwd_ffi"),                                 # cross_entropy.py:28-36
    ("ce_bwd", "nl_ce_bwd_ffi"),                                 # cross_entropy.py:39-46
    ("ce_fwd_bwd", "nl_ce_fwd_bwd_ffi"),                         # cross_entropy.py:55-65, one pass
)


def register(lib_path: str | None = None, platform: str = "ROCM") -> None:
    import jax

    lib = ctypes.cdll.LoadLibrary(lib_path or os.environ.get("NLEARN_JAX_FFI_LIB", "libnlearn_jax_ffi.so"))
    for target, symbol in TARGETS:
        jax.ffi.register_ffi_target(target, jax.ffi.pycapsule(getattr(lib, symbol)), platform=platform)
