"""HIP kernels behind nlearn's ``nlearn.kernels`` entry points (gemm, cross_entropy)."""
