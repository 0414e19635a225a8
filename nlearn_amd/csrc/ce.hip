// ce.hip — fused softmax cross-entropy for gfx950.
//
// Algorithm (nlearn/kernels/cross_entropy.py:49-81, cross_entropy.metal:38-97):
//   lse[m]  = max_v x[m,v] + log sum_v exp(x[m,v] - max)
//   loss[m] = lse[m] - x[m, t[m]]
//   dx[m,v] = (exp(x[m,v] - lse[m]) - [v == t[m]]) * scale      (scale = 1/M)
//
// MI355X design: one workgroup of 512 lanes owns one row. The whole bf16 row
// (50257 x 2 B = 100 KB) is pulled into registers with 16-byte loads, so HBM
// sees exactly one read and one write of the row: per-lane (max, sum) ->
// wavefront butterfly -> 8-wave LDS combine -> lse -> dlogits straight from
// registers, optionally written over the logits in place. Rows whose start is
// not 16-byte aligned (dense V = 50257) peel <8 head and tail elements. The
// row is streamed with nontemporal loads and stores (read once, written once).
#include "common.h"

namespace nl {
namespace {

constexpr int kCeBlock = 512;
constexpr int kCeWaves = kCeBlock / kWave;

struct RowSplit {
  int head;   // scalar elements before the first 16-byte boundary
  int nbody;  // 8-element vectors
  int tail;   // scalar elements after the body
};

__device__ __forceinline__ RowSplit split_row(const uint16_t* row, int V) {
  const int mis = (int)(((uintptr_t)row & 15) >> 1);
  int head = mis ? 8 - mis : 0;
  if (head > V) head = V;
  RowSplit r;
  r.head = head;
  r.nbody = (V - head) >> 3;
  r.tail = (V - head) & 7;
  return r;
}

// Combine two (max, sum of exp2(x*log2e - max)) partials, both in log2 units.
__device__ __forceinline__ void combine(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) {
    m = mn;
    s = 0.f;
    return;
  }
  s = s * fast_exp2(m - mn) + s2 * fast_exp2(m2 - mn);
  m = mn;
}

// Block-wide (max, sum) reduction; returns lse in natural-log units on every lane.
__device__ __forceinline__ float block_lse(float m, float s, float* sm_m, float* sm_s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o, kWave);
    const float s2 = __shfl_xor(s, o, kWave);
    combine(m, s, m2, s2);
  }
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  if (lane == 0) {
    sm_m[wave] = m;
    sm_s[wave] = s;
  }
  __syncthreads();
  float M = sm_m[0], S = sm_s[0];
#pragma unroll
  for (int w = 1; w < kCeWaves; ++w) combine(M, S, sm_m[w], sm_s[w]);
  return (M + fast_log2(S)) * kLn2;
}

// Register-resident single pass. NVEC 16-byte vectors per lane.
template <int NVEC, bool kGrad>
__global__ __launch_bounds__(kCeBlock) void ce_rowreg_kernel(
    int M, int V, const uint16_t* __restrict__ logits, int64_t ld, const int32_t* __restrict__ targets,
    float* __restrict__ loss, float* __restrict__ lse_out, float scale, uint16_t* dlogits, int64_t ldd) {
  __shared__ float sm_m[kCeWaves], sm_s[kCeWaves], sm_xt[1];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* lrow = logits + (int64_t)row * ld;
  const RowSplit rs = split_row(lrow, V);
  const u32x4* body = reinterpret_cast<const u32x4*>(lrow + rs.head);

  u32x4 v[NVEC];
#pragma unroll
  for (int j = 0; j < NVEC; ++j) {
    const int idx = j * kCeBlock + tid;
    if (idx < rs.nbody) v[j] = __builtin_nontemporal_load(body + idx);
  }
  // one optional scalar element: head (tid < head) or tail (8 <= tid < 8 + tail)
  int eidx = -1;
  if (tid < rs.head) eidx = tid;
  else if (tid >= 8 && tid < 8 + rs.tail) eidx = rs.head + rs.nbody * 8 + (tid - 8);
  const float xe = (eidx >= 0) ? bf16_to_f32(lrow[eidx]) * kLog2e : -INFINITY;

  const int t = targets[row];
  const bool tvalid = (t >= 0) && (t < V);
  if (tid == 0) sm_xt[0] = tvalid ? bf16_to_f32(lrow[t]) : __builtin_nanf("");

  // per-lane max (log2 units)
  float m = xe;
#pragma unroll
  for (int j = 0; j < NVEC; ++j) {
    if (j * kCeBlock + tid < rs.nbody) {
#pragma unroll
      for (int q = 0; q < 4; ++q) m = fmaxf(m, fmaxf(bf16_lo(v[j][q]), bf16_hi(v[j][q])) * kLog2e);
    }
  }
  // keep the row packed: without this the compiler caches all unpacked floats
  // across the three passes (2x the registers, a third of the occupancy)
#pragma unroll
  for (int j = 0; j < NVEC; ++j) asm volatile("" : "+v"(v[j]));
  float s = 0.f;
  if (m != -INFINITY) {
    s = (eidx >= 0) ? fast_exp2(xe - m) : 0.f;
#pragma unroll
    for (int j = 0; j < NVEC; ++j) {
      if (j * kCeBlock + tid < rs.nbody) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          s += fast_exp2(__builtin_fmaf(bf16_lo(v[j][q]), kLog2e, -m));
          s += fast_exp2(__builtin_fmaf(bf16_hi(v[j][q]), kLog2e, -m));
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NVEC; ++j) asm volatile("" : "+v"(v[j]));
  const float lse = block_lse(m, s, sm_m, sm_s);  // contains __syncthreads()
  if (tid == 0) {
    loss[row] = lse - sm_xt[0];
    lse_out[row] = lse;
  }
  if constexpr (kGrad) {
    uint16_t* drow = dlogits + (int64_t)row * ldd;
    u32x4* dbody = reinterpret_cast<u32x4*>(drow + rs.head);
    const float nb = -lse * kLog2e;
    // which lane/vector/element holds the target (body only; head/tail handled below)
    int own_j = -1, own_e = 0;
    if (tvalid && t >= rs.head && t < rs.head + rs.nbody * 8) {
      const int vi = (t - rs.head) >> 3;
      if ((vi % kCeBlock) == tid) {
        own_j = vi / kCeBlock;
        own_e = (t - rs.head) & 7;
      }
    }
#pragma unroll
    for (int j = 0; j < NVEC; ++j) {
      if (j * kCeBlock + tid < rs.nbody) {
        float p[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          p[2 * q] = fast_exp2(__builtin_fmaf(bf16_lo(v[j][q]), kLog2e, nb)) * scale;
          p[2 * q + 1] = fast_exp2(__builtin_fmaf(bf16_hi(v[j][q]), kLog2e, nb)) * scale;
        }
        if (j == own_j) {
#pragma unroll
          for (int e = 0; e < 8; ++e) p[e] -= (e == own_e) ? scale : 0.f;
        }
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(p[2 * q], p[2 * q + 1]);
        __builtin_nontemporal_store(o, dbody + j * kCeBlock + tid);
      }
    }
    if (eidx >= 0) {
      float p = fast_exp2(xe + nb) * scale;
      if (tvalid && eidx == t) p -= scale;
      drow[eidx] = f32_to_bf16(p);
    }
  }
}

// Generic path: any V, any alignment. Two reads of the row (the second hits L2
// for rows that fit). Used by nl_ce_bwd, and by nl_ce_fwd_bwd when the row does
// not fit in registers or when dlogits has a different alignment than logits.
template <bool kFwd, bool kGrad>
__global__ __launch_bounds__(kCeBlock) void ce_generic_kernel(
    int M, int V, const uint16_t* __restrict__ logits, int64_t ld, const int32_t* __restrict__ targets,
    float* loss, float* lse_io, float scale, uint16_t* dlogits, int64_t ldd) {
  __shared__ float sm_m[kCeWaves], sm_s[kCeWaves], sm_xt[1];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* lrow = logits + (int64_t)row * ld;
  const int t = targets[row];
  const bool tvalid = (t >= 0) && (t < V);
  float lse;
  if constexpr (kFwd) {
    if (tid == 0) sm_xt[0] = tvalid ? bf16_to_f32(lrow[t]) : __builtin_nanf("");
    float m = -INFINITY, s = 0.f;
    for (int v0 = tid; v0 < V; v0 += kCeBlock) {
      const float x = bf16_to_f32(lrow[v0]) * kLog2e;
      combine(m, s, x, 1.f);
    }
    lse = block_lse(m, s, sm_m, sm_s);
    if (tid == 0) {
      loss[row] = lse - sm_xt[0];
      lse_io[row] = lse;
    }
  } else {
    lse = lse_io[row];
  }
  if constexpr (kGrad) {
    uint16_t* drow = dlogits + (int64_t)row * ldd;
    const float nb = -lse * kLog2e;
    for (int v0 = tid; v0 < V; v0 += kCeBlock) {
      float p = fast_exp2(__builtin_fmaf(bf16_to_f32(lrow[v0]), kLog2e, nb)) * scale;
      if (v0 == t) p -= scale;
      drow[v0] = f32_to_bf16(p);
    }
  }
}

constexpr int kMeanBlock = 1024;
__global__ __launch_bounds__(kMeanBlock) void mean_kernel(const float* __restrict__ x, int n, float* out) {
  __shared__ float sm[kMeanBlock / kWave];
  float acc = 0.f;
  // eight loads in flight per thread, added in the same order as one at a time
  for (int i0 = threadIdx.x; i0 < n; i0 += 8 * kMeanBlock) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = i0 + e * kMeanBlock < n ? x[i0 + e * kMeanBlock] : 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (i0 + e * kMeanBlock < n) acc += v[e];
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & (kWave - 1)) == 0) sm[threadIdx.x / kWave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int w = 0; w < kMeanBlock / kWave; ++w) s += sm[w];
    out[0] = (n > 0) ? s / (float)n : __builtin_nanf("");
  }
}

// x *= *g in place (bf16 rows), 8 elements per lane and load when the rows
// are 16-byte aligned; a no-op when *g == 1 (every workgroup exits after one load)
__global__ __launch_bounds__(256) void scale_rows_kernel(uint16_t* x, int64_t rows, int64_t cols, int64_t ld,
                                                         const float* g) {
  const float gs = *g;
  if (gs == 1.0f) return;
  const bool vec = (ld % 8) == 0 && ((uintptr_t)x & 15) == 0;
  const int64_t c8 = vec ? cols / 8 : 0;
  const int64_t step = (int64_t)gridDim.x * 256;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    uint16_t* xr = x + r * ld;
    for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < c8; c += step) {
      u32x4 v = reinterpret_cast<const u32x4*>(xr)[c];
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = pack_bf16x2(bf16_lo(v[k]) * gs, bf16_hi(v[k]) * gs);
      reinterpret_cast<u32x4*>(xr)[c] = v;
    }
    for (int64_t c = c8 * 8 + (int64_t)blockIdx.x * 256 + threadIdx.x; c < cols; c += step)
      xr[c] = f32_to_bf16(bf16_to_f32(xr[c]) * gs);
  }
}

template <bool kGrad>
hipError_t launch_rowreg(int nvec, hipStream_t st, int M, int V, const uint16_t* lg, int64_t ld, const int32_t* tg,
                         float* loss, float* lse, float scale, uint16_t* dl, int64_t ldd) {
  dim3 grid(M), block(kCeBlock);
#define NL_CE_CASE(N)                                                                                         \
  case N:                                                                                                   \
    hipLaunchKernelGGL((ce_rowreg_kernel<N, kGrad>), grid, block, 0, st, M, V, lg, ld, tg, loss, lse, scale, \
                       dl, ldd);                                                                            \
    return hipSuccess;
  switch (nvec) {
    NL_CE_CASE(1)
    NL_CE_CASE(2)
    NL_CE_CASE(4)
    NL_CE_CASE(7)
    NL_CE_CASE(10)
    NL_CE_CASE(13)
    default: return hipErrorInvalidValue;
  }
#undef NL_CE_CASE
}

// smallest instantiated register capacity for a row of V elements (0 = none)
int pick_nvec(int V) {
  const int need = (V / 8 + 1 + kCeBlock - 1) / kCeBlock;  // body vectors per lane
  const int sizes[] = {1, 2, 4, 7, 10, 13};
  for (int s : sizes)
    if (need <= s) return s;
  return 0;
}

int check_ce_args(int M, int V, const void* logits, int64_t ld, const void* targets, const void* a, const void* b) {
  if (M < 0 || V <= 0) return nl_set_error(NL_EINVAL, "ce: need M >= 0 and V > 0");
  if (ld < V) return nl_set_error(NL_EINVAL, "ce: ld_logits < V");
  if (M > 0 && (!logits || !targets || !a || !b)) return nl_set_error(NL_EINVAL, "ce: null pointer");
  if (((uintptr_t)logits & 1) != 0) return nl_set_error(NL_EALIGN, "ce: logits not 2-byte aligned");
  return NL_OK;
}

}  // namespace
}  // namespace nl

using namespace nl;

extern "C" int nl_ce_fwd(void* stream, int M, int V, const nl_bf16* logits, int64_t ld_logits,
                         const int32_t* targets, float* loss, float* lse) {
  int rc = check_ce_args(M, V, logits, ld_logits, targets, loss, lse);
  if (rc) return rc;
  if (M == 0) return NL_OK;
  hipStream_t st = (hipStream_t)stream;
  const int nvec = pick_nvec(V);
  if (nvec) {
    launch_rowreg<false>(nvec, st, M, V, logits, ld_logits, targets, loss, lse, 0.f, nullptr, 0);
  } else {
    hipLaunchKernelGGL((ce_generic_kernel<true, false>), dim3(M), dim3(kCeBlock), 0, st, M, V, logits, ld_logits,
                       targets, loss, lse, 0.f, nullptr, 0);
  }
  return nl_check_launch("nl_ce_fwd");
}

extern "C" int nl_ce_bwd(void* stream, int M, int V, const nl_bf16* logits, int64_t ld_logits,
                         const int32_t* targets, const float* lse, float scale, nl_bf16* dlogits,
                         int64_t ld_dlogits) {
  int rc = check_ce_args(M, V, logits, ld_logits, targets, lse, dlogits);
  if (rc) return rc;
  if (ld_dlogits < V) return nl_set_error(NL_EINVAL, "ce: ld_dlogits < V");
  if (M == 0) return NL_OK;
  hipLaunchKernelGGL((ce_generic_kernel<false, true>), dim3(M), dim3(kCeBlock), 0, (hipStream_t)stream, M, V,
                     logits, ld_logits, targets, nullptr, const_cast<float*>(lse), scale, dlogits, ld_dlogits);
  return nl_check_launch("nl_ce_bwd");
}

extern "C" int nl_ce_fwd_bwd(void* stream, int M, int V, const nl_bf16* logits, int64_t ld_logits,
                             const int32_t* targets, float* loss, float* lse, float scale, nl_bf16* dlogits,
                             int64_t ld_dlogits) {
  int rc = check_ce_args(M, V, logits, ld_logits, targets, loss, lse);
  if (rc) return rc;
  if (!dlogits && M > 0) return nl_set_error(NL_EINVAL, "ce: null dlogits");
  if (ld_dlogits < V) return nl_set_error(NL_EINVAL, "ce: ld_dlogits < V");
  const bool alias = (const void*)dlogits == (const void*)logits;
  if (alias && ld_dlogits != ld_logits)
    return nl_set_error(NL_EINVAL, "ce: in-place dlogits needs ld_dlogits == ld_logits");
  if (M == 0) return NL_OK;
  hipStream_t st = (hipStream_t)stream;
  const int nvec = pick_nvec(V);
  const bool same_phase = ((((uintptr_t)logits ^ (uintptr_t)dlogits) & 15) == 0) && (ld_logits == ld_dlogits);
  if (nvec && same_phase) {
    launch_rowreg<true>(nvec, st, M, V, logits, ld_logits, targets, loss, lse, scale, dlogits, ld_dlogits);
  } else if (alias) {
    // cannot happen (alias implies same phase) unless the row exceeds the register capacity;
    // the generic kernel reads each row twice, so an in-place write would race its own reads.
    return nl_set_error(NL_EUNSUPPORTED, "ce: in-place dlogits needs V <= 53240");
  } else {
    hipLaunchKernelGGL((ce_generic_kernel<true, true>), dim3(M), dim3(kCeBlock), 0, st, M, V, logits, ld_logits,
                       targets, loss, lse, scale, dlogits, ld_dlogits);
  }
  return nl_check_launch("nl_ce_fwd_bwd");
}

extern "C" int nl_mean_f32(void* stream, const float* x, int n, float* out) {
  if (n < 0 || !out || (n > 0 && !x)) return nl_set_error(NL_EINVAL, "mean: bad arguments");
  hipLaunchKernelGGL(mean_kernel, dim3(1), dim3(kMeanBlock), 0, (hipStream_t)stream, x, n, out);
  return nl_check_launch("nl_mean_f32");
}

extern "C" int nl_scale_bf16_by_device_scalar(void* stream, nl_bf16* x, int64_t rows, int64_t cols, int64_t ld,
                                              const float* g) {
  if (rows < 0 || cols < 0 || ld < cols || !g) return nl_set_error(NL_EINVAL, "scale: bad arguments");
  if (rows == 0 || cols == 0) return NL_OK;
  if (!x) return nl_set_error(NL_EINVAL, "scale: null x");
  // a small grid-stride launch (4 workgroups per CU): it sits between the CE and
  // the LM-head dX, and when *g == 1 every workgroup exits after one load
  const int64_t gx = std::min<int64_t>((cols + 2047) / 2048, 8);
  const int64_t gy = std::min<int64_t>(rows, 128);
  hipLaunchKernelGGL(scale_rows_kernel, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, (hipStream_t)stream, x, rows,
                     cols, ld, g);
  return nl_check_launch("nl_scale_bf16_by_device_scalar");
}
