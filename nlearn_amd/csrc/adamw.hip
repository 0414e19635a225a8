// adamw.hip — fused AdamW step (fp32 master weights, fp32 moments) that also
// writes the bf16 compute copy of the weight. One HBM pass over p, g, m, v.
//
// Semantics: optax.adamw (nlearn/train.py:504-505), decoupled weight decay on
// every parameter, bias correction with the update count.
#include "common.h"

namespace nl {
namespace {

// The decay rates as the kernels use them: b and 1 - b, each rounded once to
// fp32 from the caller's double (optax computes (1 - b) * g with b a Python
// float: 1 - 0.999 in fp32 arithmetic would be 0.00099998713, not 0.001).
struct Betas {
  float b1, omb1, b2, omb2;
};
Betas make_betas(double b1, double b2) { return Betas{(float)b1, (float)(1.0 - b1), (float)b2, (float)(1.0 - b2)}; }

// One element of the update, in optax.adamw's order (scale_by_adam, then
// add_decayed_weights, then -lr): m = (1-b1) g + b1 m, v = (1-b2) g^2 + b2 v,
// p -= lr * (m/bc1 / (sqrt(v/bc2) + eps) + wd p). Every multiply-add is an
// explicit fmaf, so the rounding is fixed by the source and all kernels below
// agree bit for bit.
__device__ __forceinline__ void adam1(float gi, float& m, float& v, float& p, float lr, const Betas& bt, float eps,
                                      float wd, float inv_bc1, float inv_bc2) {
  m = __builtin_fmaf(bt.b1, m, bt.omb1 * gi);
  v = __builtin_fmaf(bt.b2, v, bt.omb2 * (gi * gi));
  const float step = (m * inv_bc1) / (__builtin_sqrtf(v * inv_bc2) + eps);
  p = __builtin_fmaf(-lr, __builtin_fmaf(wd, p, step), p);
}

__global__ __launch_bounds__(256) void adamw_kernel(int64_t rows, int64_t cols, float* __restrict__ p,
                                                    const float* __restrict__ g, float* __restrict__ m,
                                                    float* __restrict__ v, uint16_t* __restrict__ pb, int64_t ldb,
                                                    float lr, Betas bt, float eps, float wd, float bc1,
                                                    float bc2) {
  const float inv_bc1 = 1.f / bc1, inv_bc2 = 1.f / bc2;
  const int64_t n = rows * cols;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float mi = m[i], vi = v[i], pn = p[i];
    adam1(g[i], mi, vi, pn, lr, bt, eps, wd, inv_bc1, inv_bc2);
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
                                                         Betas bt, float eps, float wd, float bc1, float bc2) {
  const float inv_bc1 = 1.f / bc1, inv_bc2 = 1.f / bc2;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const f32x4 gi = g[i];
    f32x4 mi = m[i], vi = v[i], pn = p[i];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a = mi[e], b = vi[e], c = pn[e];
      adam1(gi[e], a, b, c, lr, bt, eps, wd, inv_bc1, inv_bc2);
      mi[e] = a, vi[e] = b, pn[e] = c;
    }
    m[i] = mi;
    v[i] = vi;
    p[i] = pn;
    if (pb) pb[i] = u32x2{pack_bf16x2(pn[0], pn[1]), pack_bf16x2(pn[2], pn[3])};
  }
}

constexpr int kChunk = 8192;  // elements per workgroup of the multi-tensor update

// One workgroup per chunk of kChunk elements of one leaf; the leaf is found by
// a binary search over chunk0 (the table is sorted by construction).
template <bool CLIP>
__global__ __launch_bounds__(256) void adamw_multi_kernel(int n, const nl_adamw_tensor* __restrict__ T,
                                                          const float* __restrict__ hyper, Betas bt, float eps,
                                                          float wd, const float* __restrict__ gnorm_dev,
                                                          float max_norm) {
  const int64_t chunk = blockIdx.x;
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (T[mid].chunk0 <= chunk) lo = mid;
    else hi = mid - 1;
  }
  const nl_adamw_tensor t = T[lo];
  const float lr = hyper[0], inv_bc1 = 1.f / hyper[1], inv_bc2 = 1.f / hyper[2];
  // optax.clip_by_global_norm: g unchanged while ||g|| < max_norm, else (g / ||g||) * max_norm
  const float gnorm = CLIP ? *gnorm_dev : 0.f;
  const bool clip = CLIP && !(gnorm < max_norm);
  auto clipped = [&](float g) { return clip ? (g / gnorm) * max_norm : g; };
  const int64_t numel = t.rows * t.cols;
  const int64_t e0 = (chunk - t.chunk0) * kChunk;
  const int64_t e1 = min(numel, e0 + kChunk);
  if (e0 >= e1) return;  // only with a launch larger than the prepared chunk count
  // leaves are 16-byte aligned and chunks start at multiples of 4: vec4 body, scalar tail
  const int64_t v1 = e0 + ((e1 - e0) & ~(int64_t)3);
  // p, g, m and v stream through once per step (nontemporal); the bf16 shadow
  // is read again by the next forward pass and stays cacheable. The lane's
  // (row, column) advances incrementally instead of by a 64-bit division.
  int64_t e = e0 + threadIdx.x * 4;
  int64_t r = t.shadow && t.cols > 0 ? e / t.cols : 0;
  int64_t c = e - r * t.cols;
  for (; e < v1; e += 256 * 4) {
    const f32x4 gi = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(t.g + e));
    f32x4 m = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(t.m + e));
    f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(t.v + e));
    f32x4 p = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(t.p + e));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float mk = m[k], vk = v[k], pk = p[k];
      adam1(clipped(gi[k]), mk, vk, pk, lr, bt, eps, wd, inv_bc1, inv_bc2);
      m[k] = mk, v[k] = vk, p[k] = pk;
    }
    __builtin_nontemporal_store(m, reinterpret_cast<f32x4*>(t.m + e));
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(t.v + e));
    __builtin_nontemporal_store(p, reinterpret_cast<f32x4*>(t.p + e));
    if (t.shadow) {
      const int64_t o = r * t.ld_shadow + c;
      if (c + 4 <= t.cols && (o & 3) == 0) {
        *reinterpret_cast<u32x2*>(t.shadow + o) = u32x2{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int64_t rk = (e + k) / t.cols, ck = e + k - rk * t.cols;
          t.shadow[rk * t.ld_shadow + ck] = f32_to_bf16(p[k]);
        }
      }
      c += 256 * 4;
      while (c >= t.cols) {
        c -= t.cols;
        ++r;
      }
    }
  }
  for (e = v1 + threadIdx.x; e < e1; e += 256) {
    float m = t.m[e], v = t.v[e], p = t.p[e];
    adam1(clipped(t.g[e]), m, v, p, lr, bt, eps, wd, inv_bc1, inv_bc2);
    t.m[e] = m;
    t.v[e] = v;
    t.p[e] = p;
    if (t.shadow) {
      const int64_t r = e / t.cols, c = e - r * t.cols;
      t.shadow[r * t.ld_shadow + c] = f32_to_bf16(p);
    }
  }
}

// optax.MultiSteps's running mean of micro-step gradients, with the loss-scale
// division of the reference's train_step in front of it:
//   u = g / coef[0];  acc = (coef[1] == 1) ? u : acc + (u - acc) / coef[1]
// (coef[1] = mini_step + 1; optax's acc is zero on the first micro-step, so
// its formula reduces to acc = u there). acc may equal g (in-place unscale).
__global__ __launch_bounds__(256) void grad_accumulate_kernel(int64_t n, float* acc, const float* g,
                                                              const float* __restrict__ coef) {
  const float s = coef[0], k1 = coef[1];
  const bool first = k1 == 1.f;
  const int64_t n4 = n / 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const f32x4 gi = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(g) + i);
    f32x4 a = first ? f32x4{0.f, 0.f, 0.f, 0.f} : reinterpret_cast<const f32x4*>(acc)[i];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float u = gi[k] / s;
      a[k] = first ? u : a[k] + (u - a[k]) / k1;
    }
    reinterpret_cast<f32x4*>(acc)[i] = a;
  }
  for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float u = g[i] / s;
    acc[i] = first ? u : acc[i] + (u - acc[i]) / k1;
  }
}

constexpr int kNormParts = 1024;  // partial sums of the global norm (fixed, so the order is fixed)

__device__ __forceinline__ float block_sum256(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// part[b] = sum of g[i]^2 over the elements block b visits (grid-stride, fixed order)
__global__ __launch_bounds__(256) void sumsq_partial_kernel(int64_t n, const float* __restrict__ g,
                                                            float* __restrict__ part) {
  __shared__ float red[4];
  float acc = 0.f;
  const int64_t n4 = n / 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const f32x4 x = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(g) + i);
    acc = __builtin_fmaf(x[0], x[0], acc);
    acc = __builtin_fmaf(x[1], x[1], acc);
    acc = __builtin_fmaf(x[2], x[2], acc);
    acc = __builtin_fmaf(x[3], x[3], acc);
  }
  for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    acc = __builtin_fmaf(g[i], g[i], acc);
  const float t = block_sum256(acc, red);
  if (threadIdx.x == 0) part[blockIdx.x] = t;
}

// out[0] = sqrt(sum of the partials), reduced in a fixed order
__global__ __launch_bounds__(256) void sumsq_final_kernel(int parts, const float* __restrict__ part,
                                                          float* __restrict__ out) {
  __shared__ float red[4];
  float acc = 0.f;
  for (int i = threadIdx.x; i < parts; i += 256) acc += part[i];
  const float t = block_sum256(acc, red);
  if (threadIdx.x == 0) out[0] = __builtin_sqrtf(t);
}

}  // namespace
}  // namespace nl

using namespace nl;

extern "C" int nl_grad_accumulate(void* stream, int64_t n, float* acc, const float* g, const float* coef_dev) {
  if (n < 0) return nl_set_error(NL_EINVAL, "grad_accumulate: negative size");
  if (n == 0) return NL_OK;
  if (!acc || !g || !coef_dev) return nl_set_error(NL_EINVAL, "grad_accumulate: null pointer");
  if ((((uintptr_t)acc | (uintptr_t)g) & 15) != 0)
    return nl_set_error(NL_EALIGN, "grad_accumulate: acc and g must be 16-byte aligned");
  const int64_t blocks = std::min<int64_t>((n / 4 + 255) / 256 + 1, 8192);
  hipLaunchKernelGGL(grad_accumulate_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, n, acc, g,
                     coef_dev);
  return nl_check_launch("nl_grad_accumulate");
}

extern "C" size_t nl_global_norm_ws_bytes(int64_t n) { return n > 0 ? kNormParts * sizeof(float) : 0; }

extern "C" int nl_global_norm(void* stream, int64_t n, const float* g, float* out, void* ws, size_t ws_bytes) {
  if (n < 0) return nl_set_error(NL_EINVAL, "global_norm: negative size");
  if (!out) return nl_set_error(NL_EINVAL, "global_norm: null output");
  if (n > 0 && (!g || !ws)) return nl_set_error(NL_EINVAL, "global_norm: null pointer");
  if (n > 0 && ws_bytes < nl_global_norm_ws_bytes(n))
    return nl_set_error(NL_EINVAL, "global_norm: workspace smaller than nl_global_norm_ws_bytes()");
  if (((uintptr_t)g & 15) != 0) return nl_set_error(NL_EALIGN, "global_norm: g must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  float* part = static_cast<float*>(ws);
  if (n > 0)
    hipLaunchKernelGGL(sumsq_partial_kernel, dim3(kNormParts), dim3(256), 0, st, n, g, part);
  hipLaunchKernelGGL(sumsq_final_kernel, dim3(1), dim3(256), 0, st, n > 0 ? kNormParts : 0, part, out);
  return nl_check_launch("nl_global_norm");
}

extern "C" int64_t nl_adamw_multi_prepare(int n_tensors, nl_adamw_tensor* T) {
  if (n_tensors < 0 || (n_tensors > 0 && !T)) return -(int64_t)nl_set_error(NL_EINVAL, "adamw_multi: bad table");
  int64_t chunks = 0;
  for (int i = 0; i < n_tensors; ++i) {
    if (T[i].rows < 0 || T[i].cols < 0) return -(int64_t)nl_set_error(NL_EINVAL, "adamw_multi: negative size");
    if (!T[i].p || !T[i].g || !T[i].m || !T[i].v)
      return -(int64_t)nl_set_error(NL_EINVAL, "adamw_multi: null pointer in the table");
    if ((((uintptr_t)T[i].p | (uintptr_t)T[i].g | (uintptr_t)T[i].m | (uintptr_t)T[i].v) & 15) != 0)
      return -(int64_t)nl_set_error(NL_EALIGN, "adamw_multi: p, g, m, v must be 16-byte aligned");
    if (T[i].shadow && (T[i].ld_shadow < T[i].cols || ((uintptr_t)T[i].shadow & 7) != 0))
      return -(int64_t)nl_set_error(NL_EINVAL, "adamw_multi: shadow needs ld_shadow >= cols and 8-byte alignment");
    T[i].chunk0 = chunks;
    chunks += (T[i].rows * T[i].cols + kChunk - 1) / kChunk;
  }
  return chunks;
}

extern "C" int nl_adamw_multi(void* stream, int n_tensors, const nl_adamw_tensor* tensors_dev, int64_t n_chunks,
                              const float* hyper_dev, double b1, double b2, float eps, float wd) {
  if (n_tensors < 0 || n_chunks < 0) return nl_set_error(NL_EINVAL, "adamw_multi: negative count");
  if (n_tensors == 0 || n_chunks == 0) return NL_OK;
  if (!tensors_dev || !hyper_dev) return nl_set_error(NL_EINVAL, "adamw_multi: null pointer");
  if (n_chunks > 0x7fffffff) return nl_set_error(NL_EINVAL, "adamw_multi: too many chunks");
  hipLaunchKernelGGL(adamw_multi_kernel<false>, dim3((unsigned)n_chunks), dim3(256), 0, (hipStream_t)stream,
                     n_tensors, tensors_dev, hyper_dev, make_betas(b1, b2), eps, wd, nullptr, 0.f);
  return nl_check_launch("nl_adamw_multi");
}

extern "C" int nl_adamw_multi_clip(void* stream, int n_tensors, const nl_adamw_tensor* tensors_dev, int64_t n_chunks,
                                   const float* hyper_dev, double b1, double b2, float eps, float wd,
                                   const float* gnorm_dev, float max_norm) {
  if (n_tensors < 0 || n_chunks < 0) return nl_set_error(NL_EINVAL, "adamw_multi: negative count");
  if (!(max_norm > 0.f)) return nl_set_error(NL_EINVAL, "adamw_multi_clip: max_norm must be > 0");
  if (n_tensors == 0 || n_chunks == 0) return NL_OK;
  if (!tensors_dev || !hyper_dev || !gnorm_dev) return nl_set_error(NL_EINVAL, "adamw_multi: null pointer");
  if (n_chunks > 0x7fffffff) return nl_set_error(NL_EINVAL, "adamw_multi: too many chunks");
  hipLaunchKernelGGL(adamw_multi_kernel<true>, dim3((unsigned)n_chunks), dim3(256), 0, (hipStream_t)stream,
                     n_tensors, tensors_dev, hyper_dev, make_betas(b1, b2), eps, wd, gnorm_dev, max_norm);
  return nl_check_launch("nl_adamw_multi_clip");
}

extern "C" int nl_adamw_step(void* stream, int64_t rows, int64_t cols, float* p, const float* g, float* m, float* v,
                             nl_bf16* p_bf16, int64_t ld_bf16, float lr, double b1, double b2, float eps, float wd,
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
                       (const f32x4*)g, (f32x4*)m, (f32x4*)v, (u32x2*)p_bf16, lr, make_betas(b1, b2), eps, wd,
                       bc1, bc2);
  } else {
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(adamw_kernel, dim3((unsigned)blocks), dim3(256), 0, st, rows, cols, p, g, m, v, p_bf16,
                       p_bf16 ? ld_bf16 : cols, lr, make_betas(b1, b2), eps, wd, bc1, bc2);
  }
  return nl_check_launch("nl_adamw_step");
}
