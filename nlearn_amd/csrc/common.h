// common.h — shared device helpers and host-side status plumbing for the
// gfx950 kernels. Everything here is CDNA4-specific: 64-lane wavefronts,
// MFMA bf16 fragments, fp32 <-> bf16 conversions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <algorithm>
#include <cstdlib>
#include <string>

#include "../../include/nlearn_hip.h"

namespace nl {

// ---------------------------------------------------------------------------
// vector types
// ---------------------------------------------------------------------------
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN). gfx950 lowers the
// __bf16 conversion to v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(uint16_t, b);
}
// Two floats -> one dword of bf16 (lo in bits 0-15): a single v_cvt_pk_bf16_f32
// (converting each half separately costs two conversions and a v_or).
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_cvt;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_cvt;
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_cvt){lo, hi}, bf16x2_cvt));
}

// ---------------------------------------------------------------------------
// exp2 / log2 on the transcendental unit (v_exp_f32 / v_log_f32).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------
// tanh-approximated GELU (the FFN activation) and its derivative, in the
// equivalent logistic form (1 + tanh(z)) / 2 = sigmoid(2z):
//   gelu(u)  = u * s,  s = 1 / (1 + 2^(u (k1 + k2 u^2))),
//              k1 = -2 c log2(e), k2 = -2 c a log2(e),  c = sqrt(2/pi), a = 0.044715
//   gelu'(u) = s * (1 + u (1 - s) (2c + 6ca u^2))
// One v_exp_f32 and one v_rcp_f32 per element, no IEEE divide. Saturation:
// 2^(+inf) = inf gives s = 0 and 2^(-inf) = 0 gives s = 1, so gelu is exact at
// both ends; the derivative clamps |u| <= 20, beyond which it is 0 or 1 in fp32.
// ---------------------------------------------------------------------------
constexpr float kGeluK1 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
constexpr float kGeluK2 = kGeluK1 * 0.044715f;
constexpr float kGeluD1 = 2.0f * 0.7978845608028654f;
constexpr float kGeluD2 = 6.0f * 0.7978845608028654f * 0.044715f;
__device__ __forceinline__ float gelu_sigmoid_arg(float u) {
  return 1.f + fast_exp2(u * __builtin_fmaf(kGeluK2, u * u, kGeluK1));
}
__device__ __forceinline__ float gelu_tanh(float u) {
  return u * __builtin_amdgcn_rcpf(gelu_sigmoid_arg(u));
}
__device__ __forceinline__ float gelu_tanh_grad(float u) {
  u = fminf(fmaxf(u, -20.f), 20.f);
  const float s = __builtin_amdgcn_rcpf(gelu_sigmoid_arg(u));
  const float q = __builtin_fmaf(kGeluD2, u * u, kGeluD1);
  return s * __builtin_fmaf(u * (1.f - s), q, 1.f);
}

// ---------------------------------------------------------------------------
// wavefront reductions (butterfly over all 64 lanes)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// ---------------------------------------------------------------------------
// MFMA wrappers (gfx950 bf16, fp32 accumulate)
//   32x32x16: a = 8 bf16 of row (lane%32), k = 8*(lane/32)..+7
//             b = 8 bf16 of col (lane%32), same k
//             d[r] = D[8*(r/4) + 4*(lane/32) + r%4][lane%32]
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& v) { return __builtin_bit_cast(bf16x8, v); }

// ---------------------------------------------------------------------------
// Global -> LDS DMA and transposing LDS reads
// ---------------------------------------------------------------------------
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Raw buffer resource over [p, p + bytes): loads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// 16 bytes per lane from a buffer straight into LDS: lane l lands at lds + 16 l.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)lds, 16, voff, soff, 0, 0);
}

// s_waitcnt vmcnt(n) (other counters unconstrained), n < 64
template <int N>
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// ds_read_b64_tr_b16: lane 16G+i receives element i%4 of the 8 bytes addressed by
// lanes 16G+4e+i/4, e = 0..3 (a 4x4 transpose of 16-bit elements per 16 lanes).
__device__ __forceinline__ u32x2 ds_read_tr16(const uint16_t* lds) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)lds));
}

// 8x8 transpose of 16-bit elements held as 8 rows x 4 dwords.
// in[r] holds row r: dword j = (col 2j, col 2j+1). out[c] holds column c:
// dword j = (row 2j, row 2j+1). 32 v_perm_b32.
__device__ __forceinline__ void transpose8x8_b16(const u32x4 in[8], u32x4 out[8]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int dw = c >> 1;
    // byte selectors: v_perm_b32(a, b, sel) picks bytes of {a, b} (b = bytes 0-3,
    // a = bytes 4-7). Low halfword from row 2j (source b), high from row 2j+1 (a).
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[c][j] = __builtin_amdgcn_perm(in[2 * j + 1][dw], in[2 * j][dw], sel);
    }
  }
}

}  // namespace nl

// ---------------------------------------------------------------------------
// host-side error plumbing (defined in api.hip)
// ---------------------------------------------------------------------------
int nl_set_error(int code, const std::string& msg);
int nl_check_launch(const char* what);
