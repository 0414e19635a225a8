// adamw.hip — fused AdamW step (fp32 master weights, fp32 moments) that also
// writes the bf16 compute copy of the weight. One HBM pass over p, g, m, v.
//
// Semantics: optax.adamw (nlearn/train.py:504-505), decoupled weight decay on
// every parameter, bias correction with the update count.
#include "common.h"

namespace nl {
namespace {

__global__ __launch_bounds__(256) void adamw_kernel(int64_t rows, int64_t cols, float* __restrict__ p,
                                                    const float* __restrict__ g, float* __restrict__ m,
                                                    float* __restrict__ v, uint16_t* __restrict__ pb, int64_t ldb,
                                                    float lr, float b1, float b2, float eps, float wd, float inv_bc1,
                                                    float inv_bc2) {
  const int64_t n = rows * cols;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float gi = g[i];
    const float mi = b1 * m[i] + (1.f - b1) * gi;
    const float vi = b2 * v[i] + (1.f - b2) * gi * gi;
    const float pi = p[i];
    const float upd = (mi * inv_bc1) / (sqrtf(vi * inv_bc2) + eps) + wd * pi;
    const float pn = pi - lr * upd;
    m[i] = mi;
    v[i] = vi;
    p[i] = pn;
    if (pb) {
      const int64_t r = i / cols, c = i - r * cols;
      pb[r * ldb + c] = f32_to_bf16(pn);
    }
  }
}

// Fast path: everything dense (ld_bf16 == cols or no bf16 copy), 4 elements per lane.
__global__ __launch_bounds__(256) void adamw_vec4_kernel(int64_t n4, f32x4* __restrict__ p,
                                                         const f32x4* __restrict__ g, f32x4* __restrict__ m,
                                                         f32x4* __restrict__ v, u32x2* __restrict__ pb, float lr,
                                                         float b1, float b2, float eps, float wd, float inv_bc1,
                                                         float inv_bc2) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const f32x4 gi = g[i], mo = m[i], vo = v[i], po = p[i];
    f32x4 mi, vi, pn;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      mi[e] = b1 * mo[e] + (1.f - b1) * gi[e];
      vi[e] = b2 * vo[e] + (1.f - b2) * gi[e] * gi[e];
      pn[e] = po[e] - lr * ((mi[e] * inv_bc1) / (sqrtf(vi[e] * inv_bc2) + eps) + wd * po[e]);
    }
    m[i] = mi;
    v[i] = vi;
    p[i] = pn;
    if (pb) pb[i] = u32x2{pack_bf16x2(pn[0], pn[1]), pack_bf16x2(pn[2], pn[3])};
  }
}

}  // namespace
}  // namespace nl

using namespace nl;

extern "C" int nl_adamw_step(void* stream, int64_t rows, int64_t cols, float* p, const float* g, float* m, float* v,
                             nl_bf16* p_bf16, int64_t ld_bf16, float lr, float b1, float b2, float eps, float wd,
                             float bc1, float bc2) {
  if (rows < 0 || cols < 0) return nl_set_error(NL_EINVAL, "adamw: negative size");
  if (rows == 0 || cols == 0) return NL_OK;
  if (!p || !g || !m || !v) return nl_set_error(NL_EINVAL, "adamw: null pointer");
  if (p_bf16 && ld_bf16 < cols) return nl_set_error(NL_EINVAL, "adamw: ld_bf16 < cols");
  if (!(bc1 > 0.f) || !(bc2 > 0.f)) return nl_set_error(NL_EINVAL, "adamw: bias corrections must be > 0");
  const int64_t n = rows * cols;
  hipStream_t st = (hipStream_t)stream;
  const bool dense_b = !p_bf16 || ld_bf16 == cols || rows == 1;
  const bool al16 = ((((uintptr_t)p | (uintptr_t)g | (uintptr_t)m | (uintptr_t)v) & 15) == 0) &&
                    (((uintptr_t)p_bf16 & 7) == 0);
  if (dense_b && al16 && (n % 4) == 0) {
    const int64_t n4 = n / 4;
    const int64_t blocks = std::min<int64_t>((n4 + 255) / 256, 8192);
    hipLaunchKernelGGL(adamw_vec4_kernel, dim3((unsigned)blocks), dim3(256), 0, st, n4, (f32x4*)p,
                       (const f32x4*)g, (f32x4*)m, (f32x4*)v, (u32x2*)p_bf16, lr, b1, b2, eps, wd, 1.f / bc1,
                       1.f / bc2);
  } else {
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(adamw_kernel, dim3((unsigned)blocks), dim3(256), 0, st, rows, cols, p, g, m, v, p_bf16,
                       p_bf16 ? ld_bf16 : cols, lr, b1, b2, eps, wd, 1.f / bc1, 1.f / bc2);
  }
  return nl_check_launch("nl_adamw_step");
}
