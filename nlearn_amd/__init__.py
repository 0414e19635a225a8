"""nlearn_amd — MI355X (gfx950) kernels for nlearn's training hot path.

Module layout mirrors the reference package:
  nlearn_amd.attention               <- nlearn/attention.py
  nlearn_amd.kernels.gemm            <- nlearn/kernels/gemm.py
  nlearn_amd.kernels.cross_entropy   <- nlearn/kernels/cross_entropy.py
  nlearn_amd.model / nlearn_amd.train <- the callers (nlearn/model.py, nlearn/train.py)
All compute goes through libnlearn_hip.so (C ABI: include/nlearn_hip.h).
"""
__version__ = "0.1.0"
