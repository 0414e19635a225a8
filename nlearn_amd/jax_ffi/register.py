"""Register the reference's jax.ffi targets with the handlers of nlearn_jax_ffi.cc.

On a JAX-ROCm install, after building ``libnlearn_jax_ffi.so`` (see the header
of nlearn_jax_ffi.cc), call ``register()`` once at import in nlearn's
``attention.py``, ``kernels/gemm.py`` and ``kernels/cross_entropy.py`` (beside
their ``ffi_call`` sites). JAX is not installed in this repository's image;
nothing here runs in its tests except ``TARGETS`` and ``CALL_SITES`` being
checked against the handlers the C++ file defines.
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

# What XLA hands each handler once the reference's wrappers carry the edits
# that bind them (bf16 operands and results; L, D, loss, lse and the GEMM's C
# in f32). Per target: (operands, results), each a tuple of (XLA FFI dtype,
# the reference line that fixes it as edited). Reference lines:
#   attention.py:97,104   Qf, Kf, Vf = x.astype(jnp.bfloat16)        (was float32)
#   attention.py:115      dOf = dO.astype(jnp.bfloat16)               (was float32)
#   attention.py:116      D = jnp.sum(dOf.astype(jnp.float32) * O.astype(jnp.float32), axis=-1)
#   attention.py:88       O result  ShapeDtypeStruct(..., jnp.bfloat16) (was float32)
#   attention.py:89       L result  float32, unchanged
#   attention.py:119      dQ result bfloat16 (was float32)
#   attention.py:124-125  dK, dV results bfloat16 (was float32)
#   gemm.py:51-52         Af, Bf bfloat16, unchanged; gemm.py:38 C float32, unchanged
#   cross_entropy.py:76   lg = ....astype(jnp.bfloat16)               (was float32)
#   cross_entropy.py:77   tg int32, unchanged
#   cross_entropy.py:33-34 loss, lse results float32, unchanged
#   cross_entropy.py:44   dlogits result bfloat16 (was float32)
#   cross_entropy.py:65   (g * dlogits).astype(dlogits.dtype): the cotangent keeps
#                         the primal logits' dtype, as custom_vjp requires
_FWD_QKV = (("BF16", "attention.py:97"), ("BF16", "attention.py:97"), ("BF16", "attention.py:97"))
_BWD_IN = (("BF16", "attention.py:104"), ("BF16", "attention.py:104"), ("BF16", "attention.py:104"),
           ("BF16", "attention.py:115"), ("F32", "attention.py:89"), ("F32", "attention.py:116"))
CALL_SITES = {
    "flash_attention_fwd": (_FWD_QKV, (("BF16", "attention.py:88"), ("F32", "attention.py:89"))),
    "flash_attention_bwd_dq": (_BWD_IN, (("BF16", "attention.py:119"),)),
    "flash_attention_bwd_dkdv": (_BWD_IN, (("BF16", "attention.py:124"), ("BF16", "attention.py:125"))),
    "gemm": ((("BF16", "gemm.py:51"), ("BF16", "gemm.py:52")), (("F32", "gemm.py:38"),)),
    "gemm_nt": ((("BF16", "gemm.py:51"), ("BF16", "gemm.py:52")), (("F32", "gemm.py:38"),)),
    "gemm_tn": ((("BF16", "gemm.py:51"), ("BF16", "gemm.py:52")), (("F32", "gemm.py:38"),)),
    "ce_fwd": ((("BF16", "cross_entropy.py:76"), ("S32", "cross_entropy.py:77")),
               (("F32", "cross_entropy.py:33"), ("F32", "cross_entropy.py:34"))),
    "ce_bwd": ((("BF16", "cross_entropy.py:76"), ("S32", "cross_entropy.py:77"), ("F32", "cross_entropy.py:34")),
               (("BF16", "cross_entropy.py:44"),)),
    "ce_fwd_bwd": ((("BF16", "cross_entropy.py:76"), ("S32", "cross_entropy.py:77")),
                   (("F32", "cross_entropy.py:33"), ("F32", "cross_entropy.py:34"), ("BF16", "cross_entropy.py:44"))),
}

# reference result declarations (jax.ShapeDtypeStruct lines) whose dtype the
# edits change to bfloat16; every other one stays float32
EDITED_RESULTS = {"attention.py:88", "attention.py:119", "attention.py:124", "attention.py:125",
                  "cross_entropy.py:44"}


def register(lib_path: str | None = None, platform: str = "ROCM") -> None:
    import jax

    lib = ctypes.cdll.LoadLibrary(lib_path or os.environ.get("NLEARN_JAX_FFI_LIB", "libnlearn_jax_ffi.so"))
    for target, symbol in TARGETS:
        jax.ffi.register_ffi_target(target, jax.ffi.pycapsule(getattr(lib, symbol)), platform=platform)
