// gemm.hip — bf16 GEMM with fp32 accumulation on gfx950 MFMA.
//
//   C[M,N] = alpha * s * op(A) . op(B) + beta * C      (s = *alpha_dev or 1)
//
// Reference semantics: nlearn/kernels/gemm.py:43-79 (bf16 operands, f32
// accumulate, forward A.B, backward dA = dC.B^T and dB = A^T.dC) and
// iree_metal/kernels/gemm.metal:48-115 (f32 accumulator per output).
//
// MI355X design
//   * v_mfma_f32_32x32x16_bf16: each wave owns a (BM/WM) x (BN/WN) sub-tile
//     held as FM x FN fp32 32x32 accumulators (AGPR-resident).
//   * Both operands are staged in LDS as [row][k] with k contiguous, 64 k per
//     stage, in a 16-byte-chunk XOR swizzle: chunk kc of row R lives at slot
//     kc ^ ((R ^ R>>3) & 7). Fragment reads (8 consecutive rows, same chunk),
//     row-contiguous writes and transposed writes are all conflict-free.
//   * An operand whose contraction dim is strided in memory (B of the forward
//     x.W, both operands of the weight gradient X^T.dY) is read as 8x8 bf16
//     blocks with 16-byte loads and transposed in registers (v_perm_b32) before
//     its LDS store, so no transposed copy is ever written to HBM.
//   * Register-prefetch + LDS double buffer: the next stage's global loads are
//     in flight while the MFMAs consume the current stage; one barrier/stage.
//   * MFMA operands are swapped (B fragment as src A) so every lane ends up
//     with 4 consecutive output columns: 16-byte fp32 / 8-byte bf16 stores.
//   * M, N and K tails are masked in-kernel (zero-filled loads, guarded stores).
#include "common.h"

namespace nl {
namespace {

constexpr int BK = 64;            // k per LDS stage
constexpr int CHUNKS = BK / 8;    // 16-byte chunks per staged row

struct GemmArgs {
  int M, N, K;
  const uint16_t* A;
  int64_t lda;
  const uint16_t* B;
  int64_t ldb;
  void* C;
  int64_t ldc;
  float alpha, beta;
  const float* alpha_dev;
  // split-K: workgroup b handles tile b % tiles over k in [split*k_chunk, +k_chunk)
  int tiles;
  int k_chunk;
  float* ws;      // fp32 partials [split][M][ldw] when splitting, else null
  int64_t ldw;
};

__device__ __forceinline__ int swz(int row, int kc) { return (kc ^ ((row ^ (row >> 3)) & 7)); }

// Load 8 contiguous bf16 (16 bytes) at p, zero-filling elements with index >= lim.
__device__ __forceinline__ u32x4 load8(const uint16_t* p, int lim) {
  if (lim >= 8) return *reinterpret_cast<const u32x4*>(p);
  u32x4 r = {0u, 0u, 0u, 0u};
  if (lim > 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (e < lim) {
        const uint32_t h = p[e];
        r[e >> 1] |= (e & 1) ? (h << 16) : h;
      }
    }
  }
  return r;
}

// Stage loader for one operand tile of ROWS (m or n) x BK (k).
//   KMAJ:  element (row, k) at P[row * ld + k]   (k contiguous)
//   !KMAJ: element (row, k) at P[k * ld + row]   (row contiguous)
template <int ROWS, int NT, bool KMAJ>
struct TileLoader {
  // K-major: ROWS*CHUNKS chunks; MN-major: (BK/8)*(ROWS/8) 8x8 blocks (8 loads each)
  static constexpr int UNITS = KMAJ ? ROWS * CHUNKS : (BK / 8) * (ROWS / 8);
  static constexpr int PER = (UNITS + NT - 1) / NT;
  static constexpr int REGS = KMAJ ? PER : PER * 8;
  u32x4 r[REGS];

  __device__ __forceinline__ void load(const uint16_t* __restrict__ P, int64_t ld, int row0, int rows_lim, int k0,
                                       int k_lim, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = i * NT + tid;
      if (UNITS % NT == 0 || u < UNITS) {
        if constexpr (KMAJ) {
          const int row = u / CHUNKS, kc = u % CHUNKS;
          const int grow = row0 + row, gk = k0 + kc * 8;
          if (grow < rows_lim) r[i] = load8(P + (int64_t)grow * ld + gk, k_lim - gk);
          else r[i] = u32x4{0u, 0u, 0u, 0u};
        } else {
          const int kb = u / (ROWS / 8), rb = u % (ROWS / 8);
          const int grow = row0 + rb * 8;
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const int gk = k0 + kb * 8 + q;
            if (gk < k_lim) r[i * 8 + q] = load8(P + (int64_t)gk * ld + grow, rows_lim - grow);
            else r[i * 8 + q] = u32x4{0u, 0u, 0u, 0u};
          }
        }
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t* __restrict__ S, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = i * NT + tid;
      if (UNITS % NT == 0 || u < UNITS) {
        if constexpr (KMAJ) {
          const int row = u / CHUNKS, kc = u % CHUNKS;
          *reinterpret_cast<u32x4*>(S + row * BK + swz(row, kc) * 8) = r[i];
        } else {
          const int kb = u / (ROWS / 8), rb = u % (ROWS / 8);
          u32x4 t[8];
          transpose8x8_b16(&r[i * 8], t);
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const int row = rb * 8 + c;
            *reinterpret_cast<u32x4*>(S + row * BK + swz(row, kb) * 8) = t[c];
          }
        }
      }
    }
  }
};

template <typename OutT>
__device__ __forceinline__ void store4(OutT* c, float v0, float v1, float v2, float v3);
template <>
__device__ __forceinline__ void store4<float>(float* c, float v0, float v1, float v2, float v3) {
  *reinterpret_cast<f32x4*>(c) = f32x4{v0, v1, v2, v3};
}
template <>
__device__ __forceinline__ void store4<uint16_t>(uint16_t* c, float v0, float v1, float v2, float v3) {
  *reinterpret_cast<u32x2*>(c) = u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
}
template <typename OutT>
__device__ __forceinline__ float load1(const OutT* c);
template <>
__device__ __forceinline__ float load1<float>(const float* c) { return *c; }
template <>
__device__ __forceinline__ float load1<uint16_t>(const uint16_t* c) { return bf16_to_f32(*c); }
template <typename OutT>
__device__ __forceinline__ void store1(OutT* c, float v);
template <>
__device__ __forceinline__ void store1<float>(float* c, float v) { *c = v; }
template <>
__device__ __forceinline__ void store1<uint16_t>(uint16_t* c, float v) { *c = f32_to_bf16(v); }

template <int BM, int BN, int WM, int WN, bool A_KMAJ, bool B_KMAJ, typename OutT>
__global__ __launch_bounds__(WM* WN * 64) void gemm_kernel(GemmArgs g) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  static_assert(FM >= 1 && FN >= 1, "wave tile must be >= 32x32");

  __shared__ __attribute__((aligned(16))) uint16_t smem[2][(BM + BN) * BK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int tiles_n = (g.N + BN - 1) / BN;
  const int split = blockIdx.x / g.tiles;
  const int tile = blockIdx.x - split * g.tiles;
  const int tm = tile / tiles_n, tn = tile % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = split * g.k_chunk;
  const int kend = min(g.K, kbeg + g.k_chunk);

  TileLoader<BM, NT, A_KMAJ> la;
  TileLoader<BN, NT, B_KMAJ> lb;

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
  if (nk > 0) {
    la.load(g.A, g.lda, m0, g.M, kbeg, kend, tid);
    lb.load(g.B, g.ldb, n0, g.N, kbeg, kend, tid);
    la.store(smem[0], tid);
    lb.store(smem[0] + BM * BK, tid);
    __syncthreads();
  }

  const int frow = lane & 31;   // row within a 32-row fragment
  const int fkc = lane >> 5;    // which 8-k half of a 16-k step

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const bool more = (kt + 1) < nk;
    if (more) {
      la.load(g.A, g.lda, m0, g.M, kbeg + (kt + 1) * BK, kend, tid);
      lb.load(g.B, g.ldb, n0, g.N, kbeg + (kt + 1) * BK, kend, tid);
    }
    const uint16_t* As = smem[buf];
    const uint16_t* Bs = smem[buf] + BM * BK;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int kc = ks * 2 + fkc;
      bf16x8 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * WTM + i * 32 + frow;
        af[i] = as_bf16x8(*reinterpret_cast<const u32x4*>(As + row * BK + swz(row, kc) * 8));
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int row = wn * WTN + j * 32 + frow;
        bfr[j] = as_bf16x8(*reinterpret_cast<const u32x4*>(Bs + row * BK + swz(row, kc) * 8));
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma32(bfr[j], af[i], acc[i][j]);
    }
    if (more) {
      la.store(smem[buf ^ 1], tid);
      lb.store(smem[buf ^ 1] + BM * BK, tid);
    }
    __syncthreads();
  }

  const int g4 = (lane >> 5) * 4;
  if (g.ws) {  // split-K partial: raw fp32 sums, reduced by splitk_reduce_kernel
    float* W = g.ws + (int64_t)split * g.M * g.ldw;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = m0 + wm * WTM + i * 32 + frow;
      if (m >= g.M) continue;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n0 + wn * WTN + j * 32 + q * 8 + g4;
          if (n < g.N)  // ldw is a multiple of 4 >= N: the 4-wide store stays in the row
            *reinterpret_cast<f32x4*>(W + (int64_t)m * g.ldw + n) =
                f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        }
    }
    return;
  }
  // epilogue: lane holds C[m][n..n+3] for m = row of lane, n = 8q + 4*(lane/32)
  float s = g.alpha;
  if (g.alpha_dev) s *= *g.alpha_dev;
  OutT* C = reinterpret_cast<OutT*>(g.C);
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = m0 + wm * WTM + i * 32 + frow;
    if (m >= g.M) continue;
    OutT* crow = C + (int64_t)m * g.ldc;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * WTN + j * 32 + q * 8 + g4;
        float v0 = acc[i][j][4 * q + 0] * s, v1 = acc[i][j][4 * q + 1] * s;
        float v2 = acc[i][j][4 * q + 2] * s, v3 = acc[i][j][4 * q + 3] * s;
        if (n + 4 <= g.N) {
          if (g.beta != 0.f) {
            v0 += g.beta * load1(crow + n + 0);
            v1 += g.beta * load1(crow + n + 1);
            v2 += g.beta * load1(crow + n + 2);
            v3 += g.beta * load1(crow + n + 3);
          }
          store4(crow + n, v0, v1, v2, v3);
        } else {
          const float vv[4] = {v0, v1, v2, v3};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (n + e < g.N) {
              float v = vv[e];
              if (g.beta != 0.f) v += g.beta * load1(crow + n + e);
              store1(crow + n + e, v);
            }
          }
        }
      }
    }
  }
}

// beta*C for the degenerate K == 0 case is handled by the main kernel (nk = 0).

// C = alpha * s * sum_split ws[split] + beta * C, summed in split order (deterministic).
template <typename OutT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs g, int splits) {
  const int64_t groups_n = (g.N + 3) / 4;
  const int64_t total = (int64_t)g.M * groups_n;
  float s = g.alpha;
  if (g.alpha_dev) s *= *g.alpha_dev;
  OutT* C = reinterpret_cast<OutT*>(g.C);
  const int64_t plane = (int64_t)g.M * g.ldw;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / groups_n;
    const int n = (int)(i - m * groups_n) * 4;
    const float* w = g.ws + m * g.ldw + n;
    f32x4 acc = *reinterpret_cast<const f32x4*>(w);
    for (int sp = 1; sp < splits; ++sp) {
      const f32x4 p = *reinterpret_cast<const f32x4*>(w + sp * plane);
      acc[0] += p[0];
      acc[1] += p[1];
      acc[2] += p[2];
      acc[3] += p[3];
    }
    OutT* crow = C + m * g.ldc;
    if (n + 4 <= g.N) {
      float v[4] = {acc[0] * s, acc[1] * s, acc[2] * s, acc[3] * s};
      if (g.beta != 0.f)
        for (int e = 0; e < 4; ++e) v[e] += g.beta * load1(crow + n + e);
      store4(crow + n, v[0], v[1], v[2], v[3]);
    } else {
      for (int e = 0; e < 4 && n + e < g.N; ++e) {
        float v = acc[e] * s;
        if (g.beta != 0.f) v += g.beta * load1(crow + n + e);
        store1(crow + n + e, v);
      }
    }
  }
}

// Tile configuration and K split of one product (shared by the workspace query).
struct Plan {
  int big;     // 1: 256x256 tiles, 0: 128x128
  int tiles;
  int splits;
  int k_chunk;
  int64_t ldw;
  size_t ws_bytes;
};

Plan make_plan(int M, int N, int K) {
  Plan p;
  const int64_t t256 = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
  p.big = t256 >= 512;
  const int bm = p.big ? 256 : 128;
  p.tiles = (int)((int64_t)((M + bm - 1) / bm) * ((N + bm - 1) / bm));
  p.splits = 1;
  p.k_chunk = K > 0 ? K : 1;
  // skinny outputs with a long reduction (weight gradients, K = tokens): split K
  // until ~640 workgroups are in flight, keeping >= 512 k per split
  if (p.tiles < 256 && K >= 1024) {
    int want = (640 + p.tiles - 1) / p.tiles;
    int maxs = K / 512;
    int sp = want < maxs ? want : maxs;
    if (sp > 1) {
      int chunk = (K + sp - 1) / sp;
      chunk = (chunk + BK - 1) / BK * BK;
      p.k_chunk = chunk;
      p.splits = (K + chunk - 1) / chunk;
    }
  }
  p.ldw = ((int64_t)N + 7) / 8 * 8;
  p.ws_bytes = p.splits > 1 ? (size_t)p.splits * M * p.ldw * sizeof(float) : 0;
  return p;
}

template <int BM, int BN, int WM, int WN, bool AK, bool BK_, typename OutT>
void launch_cfg(GemmArgs g, const Plan& p, hipStream_t st) {
  g.tiles = p.tiles;
  g.k_chunk = p.k_chunk;
  if (p.splits > 1) {
    g.ldw = p.ldw;  // g.ws already set by the caller
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, AK, BK_, OutT>), dim3(p.tiles * p.splits), dim3(WM * WN * 64),
                       0, st, g);
    const int64_t work = (int64_t)g.M * ((g.N + 3) / 4);
    const int blocks = (int)std::min<int64_t>((work + 255) / 256, 4096);
    hipLaunchKernelGGL((splitk_reduce_kernel<OutT>), dim3(blocks), dim3(256), 0, st, g, p.splits);
  } else {
    g.ws = nullptr;
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, AK, BK_, OutT>), dim3(p.tiles), dim3(WM * WN * 64), 0, st, g);
  }
}

template <bool AK, bool BK_, typename OutT>
void launch_layout(const GemmArgs& g, const Plan& p, hipStream_t st) {
  if (p.big) launch_cfg<256, 256, 2, 2, AK, BK_, OutT>(g, p, st);
  else launch_cfg<128, 128, 2, 2, AK, BK_, OutT>(g, p, st);
}

template <typename OutT>
void launch_typed(int opA, int opB, const GemmArgs& g, const Plan& p, hipStream_t st) {
  // A is k-major when not transposed; B is k-major when transposed.
  if (opA == NL_OP_N && opB == NL_OP_N) launch_layout<true, false, OutT>(g, p, st);
  else if (opA == NL_OP_N && opB == NL_OP_T) launch_layout<true, true, OutT>(g, p, st);
  else if (opA == NL_OP_T && opB == NL_OP_N) launch_layout<false, false, OutT>(g, p, st);
  else launch_layout<false, true, OutT>(g, p, st);
}

}  // namespace
}  // namespace nl

using namespace nl;

extern "C" size_t nl_gemm_ws_bytes(int opA, int opB, int M, int N, int K) {
  (void)opA;
  (void)opB;
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return make_plan(M, N, K).ws_bytes;
}

extern "C" int nl_gemm_ex(void* stream, int opA, int opB, int M, int N, int K, float alpha, const nl_bf16* A,
                          int64_t lda, const nl_bf16* B, int64_t ldb, float beta, void* C, int c_dtype, int64_t ldc,
                          const float* alpha_dev, void* ws, size_t ws_bytes) {
  if (opA != NL_OP_N && opA != NL_OP_T) return nl_set_error(NL_EINVAL, "gemm: opA must be NL_OP_N or NL_OP_T");
  if (opB != NL_OP_N && opB != NL_OP_T) return nl_set_error(NL_EINVAL, "gemm: opB must be NL_OP_N or NL_OP_T");
  if (c_dtype != NL_DTYPE_F32 && c_dtype != NL_DTYPE_BF16) return nl_set_error(NL_EINVAL, "gemm: bad c_dtype");
  if (M < 0 || N < 0 || K < 0) return nl_set_error(NL_EINVAL, "gemm: negative dimension");
  if (M == 0 || N == 0) return NL_OK;
  // stored row lengths of each operand
  const int64_t a_cols = (opA == NL_OP_N) ? K : M;
  const int64_t b_cols = (opB == NL_OP_N) ? N : K;
  if (K > 0 && (lda < a_cols || ldb < b_cols)) return nl_set_error(NL_EINVAL, "gemm: leading dimension too small");
  if (ldc < N) return nl_set_error(NL_EINVAL, "gemm: ldc < N");
  if (!C || (K > 0 && (!A || !B))) return nl_set_error(NL_EINVAL, "gemm: null pointer");
  if ((((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) & 15) != 0)
    return nl_set_error(NL_EALIGN, "gemm: A, B and C must be 16-byte aligned");
  if (((lda | ldb | ldc) & 7) != 0) return nl_set_error(NL_EALIGN, "gemm: lda, ldb, ldc must be multiples of 8");
  if ((int64_t)M * N > ((int64_t)1 << 40)) return nl_set_error(NL_EINVAL, "gemm: output too large");

  GemmArgs g;
  g.M = M;
  g.N = N;
  g.K = K;
  g.A = A;
  g.lda = lda;
  g.B = B;
  g.ldb = ldb;
  g.C = C;
  g.ldc = ldc;
  g.alpha = alpha;
  g.beta = beta;
  g.alpha_dev = alpha_dev;
  Plan p = make_plan(M, N, K);
  if (p.splits > 1 && (!ws || ws_bytes < p.ws_bytes || ((uintptr_t)ws & 15) != 0)) {
    // no (usable) workspace: one workgroup per tile over the whole K range
    p.splits = 1;
    p.k_chunk = K > 0 ? K : 1;
    p.ws_bytes = 0;
  }
  g.ws = static_cast<float*>(ws);
  hipStream_t st = (hipStream_t)stream;
  if (c_dtype == NL_DTYPE_F32) launch_typed<float>(opA, opB, g, p, st);
  else launch_typed<uint16_t>(opA, opB, g, p, st);
  return nl_check_launch("nl_gemm");
}

extern "C" int nl_gemm(void* stream, int opA, int opB, int M, int N, int K, float alpha, const nl_bf16* A,
                       int64_t lda, const nl_bf16* B, int64_t ldb, float beta, void* C, int c_dtype, int64_t ldc,
                       const float* alpha_dev) {
  return nl_gemm_ex(stream, opA, opB, M, N, K, alpha, A, lda, B, ldb, beta, C, c_dtype, ldc, alpha_dev, nullptr, 0);
}
