// gemm.hip — bf16 GEMM with fp32 accumulation on gfx950 MFMA.
//
//   C[M,N] = alpha * s * op(A) . op(B) + beta * C      (s = *alpha_dev or 1)
//
// Reference semantics: nlearn/kernels/gemm.py:43-79 (bf16 operands, f32
// accumulate, forward A.B, backward dA = dC.B^T and dB = A^T.dC) and
// iree_metal/kernels/gemm.metal:48-115 (f32 accumulator per output).
//
// MI355X design (main path, gemm2_kernel)
//   * 128 x 128 output tile per workgroup of 4 waves (2 x 2), each wave a 64 x 64
//     block of fp32 32x32 MFMA accumulators (v_mfma_f32_32x32x16_bf16).
//   * Operand tiles go global -> LDS with buffer_load_dwordx4 ... lds (LDS DMA):
//     no staging registers and no ds_write; per-lane offsets are fixed for the
//     whole K loop and the K advance is a scalar offset. The buffer range check
//     clips rows past the matrix (no edge branches in the loop).
//   * An operand whose contraction dim is contiguous is stored [row][k] in LDS
//     with a 16-byte-chunk XOR swizzle and read with ds_read_b128; an operand
//     whose contraction dim is strided (B of the forward x.W, both operands of
//     the weight gradient X^T.dY) stays [k][row] as in memory and is read with
//     ds_read_b64_tr_b16, the gfx950 transposing LDS read. Nothing is ever
//     transposed in HBM or in registers.
//   * Double-buffered LDS stages of 64 k, one barrier per stage. A k-contiguous
//     operand then arrives in 128-byte pieces of each row: when the previous
//     kernel has just written it, it comes from DRAM, where 64-byte pieces
//     (32-k stages) ran a third slower.
//   * 256 x 256 tiles (8 waves, the LM head) bound by the CU's global -> LDS
//     path; in the weight-gradient (TN) form half of the waves issue each
//     stage's DMA, so one wave per SIMD computes while the other queues loads.
//   * Workgroup ids are remapped so each XCD (own L2) walks a contiguous run of
//     tiles in groups of 8 M-tiles, sharing A and B panels in its L2.
//   * Small outputs with a long reduction (weight gradients) split K across
//     workgroups into fp32 partials reduced in a fixed order (deterministic).
//   * MFMA operands are swapped (B fragment as src A) so every lane ends up with
//     4 consecutive output columns: 16-byte fp32 / 8-byte bf16 stores.
//   * A ragged K tail is staged through registers with element masks.
//   * Operands beyond the 2 GB reach of 32-bit buffer offsets are split on the
//     host into sub-products that fit it (panels of M or N; chunks of K summed
//     in the fp32 output).
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
  // fused epilogue (NL_EPI_*): bias[N] fp32, aux [M][ldaux] bf16
  int epi;
  const float* bias;
  uint16_t* aux;
  int64_t ldaux;
  // cross-entropy epilogues of the fused LM head (kEpiCeStats, kEpiCeGrad):
  // column n of the product is vocabulary entry ce_v0 + n.
  const int32_t* ce_tgt;   // targets [M]
  const float* ce_lse;     // logsumexp [M] (gradient)
  float* ce_part;          // per-row, per-tile (max, sum) partials [M][tiles_n] (statistics)
  float* ce_correct;       // the target's logit [M] (statistics)
  int ce_v0;
  float ce_scale;          // gradient scale (times *ce_scale_dev when given)
  const float* ce_scale_dev;
};

// Epilogues of the fused LM head + cross-entropy (internal; not NL_EPI_* values).
// Both see the logits l = bf16(alpha * s * acc), the values the unfused path
// stores and the CE kernel reads.
//   kEpiCeStats: nothing is stored; each row of a tile yields (max, sum of
//                2^(l*log2e - max)) over the tile's columns and, from the
//                tile holding it, the target's logit.
//   kEpiCeGrad:  C = bf16((exp(l - lse[m]) - [v0 + n == t[m]]) * scale).
constexpr int kEpiCeStats = 16;
constexpr int kEpiCeGrad = 17;

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

// Output of one lane's 4 consecutive columns C[m][n..n+3] (v = alpha * s * acc):
//   NL_EPI_BIAS       v += b[0..3]                          (then + beta * C)
//   NL_EPI_BIAS_GELU  u = bf16(v + b[0..3]); aux = u; C = gelu(u)
//   NL_EPI_DGELU      C = v * gelu'(a[0..3])                (a = the saved u)
// b = bias[n..n+3], a = aux[m][n..n+3], already fetched by the caller (entries
// at or beyond N are unspecified). Columns at or beyond N are not written.
template <typename OutT, int EPI>
__device__ __forceinline__ void epilogue_apply(const GemmArgs& g, int64_t m, int n, float v[4], const f32x4& b,
                                               const u32x2& a) {
  OutT* crow = reinterpret_cast<OutT*>(g.C) + m * g.ldc;
  const bool full = n + 4 <= g.N;
  if constexpr (EPI == NL_EPI_BIAS || EPI == NL_EPI_BIAS_GELU) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += b[e];
  }
  if constexpr (EPI == NL_EPI_BIAS_GELU) {
    uint16_t* arow = g.aux + m * g.ldaux;
    uint16_t u[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      u[e] = f32_to_bf16(v[e]);
      v[e] = gelu_tanh(bf16_to_f32(u[e]));
    }
    if (full) {
      *reinterpret_cast<u32x2*>(arow + n) =
          u32x2{(uint32_t)u[0] | ((uint32_t)u[1] << 16), (uint32_t)u[2] | ((uint32_t)u[3] << 16)};
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < g.N) arow[n + e] = u[e];
    }
  } else if constexpr (EPI == NL_EPI_DGELU) {
    v[0] *= gelu_tanh_grad(bf16_lo(a[0]));
    v[1] *= gelu_tanh_grad(bf16_hi(a[0]));
    v[2] *= gelu_tanh_grad(bf16_lo(a[1]));
    v[3] *= gelu_tanh_grad(bf16_hi(a[1]));
  }
  // the GELU forms are validated to have beta == 0
  const bool use_beta = (EPI == NL_EPI_NONE || EPI == NL_EPI_BIAS) && g.beta != 0.f;
  if (full) {
    if (use_beta) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += g.beta * load1(crow + n + e);
    }
    store4(crow + n, v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (n + e < g.N) {
        float x = v[e];
        if (use_beta) x += g.beta * load1(crow + n + e);
        store1(crow + n + e, x);
      }
    }
  }
}

// Epilogue with its operands fetched from global memory, dispatching on g.epi
// (the split-K reduction).
template <typename OutT>
__device__ __forceinline__ void epilogue4_any(const GemmArgs& g, int64_t m, int n, float v[4]) {
  const bool full = n + 4 <= g.N;
  f32x4 b = {0.f, 0.f, 0.f, 0.f};
  u32x2 a = {0u, 0u};
  if (g.epi == NL_EPI_BIAS || g.epi == NL_EPI_BIAS_GELU) {
    if (full) b = *reinterpret_cast<const f32x4*>(g.bias + n);
    else
      for (int e = 0; e < 4; ++e) b[e] = n + e < g.N ? g.bias[n + e] : 0.f;
  }
  if (g.epi == NL_EPI_DGELU) {
    const uint16_t* arow = g.aux + m * g.ldaux;
    if (full) a = *reinterpret_cast<const u32x2*>(arow + n);
    else {
      uint16_t t[4] = {0, 0, 0, 0};
      for (int e = 0; e < 4; ++e)
        if (n + e < g.N) t[e] = arow[n + e];
      a = u32x2{(uint32_t)t[0] | ((uint32_t)t[1] << 16), (uint32_t)t[2] | ((uint32_t)t[3] << 16)};
    }
  }
  switch (g.epi) {
    case NL_EPI_BIAS: epilogue_apply<OutT, NL_EPI_BIAS>(g, m, n, v, b, a); break;
    case NL_EPI_BIAS_GELU: epilogue_apply<OutT, NL_EPI_BIAS_GELU>(g, m, n, v, b, a); break;
    case NL_EPI_DGELU: epilogue_apply<OutT, NL_EPI_DGELU>(g, m, n, v, b, a); break;
    default: epilogue_apply<OutT, NL_EPI_NONE>(g, m, n, v, b, a); break;
  }
}

// ===========================================================================
// v2 main loop: LDS DMA + transposing LDS reads
//
//   * Global -> LDS with buffer_load_dwordx4 ... lds: no staging registers, no
//     ds_write. Per-lane byte offsets are fixed for the whole K loop; the K
//     advance is a scalar soffset. The buffer's num_records clips rows past
//     the matrix (they read as zero, so no edge branches).
//   * K-major tile (rows x 64 k): [row][k] with the 16-byte-chunk XOR swizzle
//     of the v1 kernel; MFMA fragments are single ds_read_b128.
//   * MN-major tile (64 k x rows): stored as it sits in memory, [k][row], with
//     chunk c of k-row k at slot c ^ mnswz(k); an MFMA fragment (8 k of one
//     row) is two ds_read_b64_tr_b16, which deliver 4 consecutive k of a column
//     to each lane of a 16-lane group. No register transposes at all.
//   * A ragged K tail (K % 64 != 0) is staged once through registers with
//     element masks into the same layouts.
// ===========================================================================

// K-major tiles keep CH = BKT/8 16-byte chunks per row; chunk kc of row r sits
// at slot kc ^ kswz(r). Eight consecutive rows at one chunk (a fragment read)
// land on distinct banks for CH = 8 and CH = 4.
template <int CH>
__device__ __forceinline__ int kswz(int r) {
  if constexpr (CH == 8) return (r ^ (r >> 3)) & 7;
  else return (r >> 1) & 3;
}

// Chunk swizzle of MN-major tiles. A transposing fragment read (32 lanes per
// LDS cycle) touches chunks c0 + {0..3} of k-rows k0 + {0..3}; XOR with
// 4 (k & 3) maps those 16 (chunk, k) pairs to 16 distinct slots mod 16, i.e.
// all 64 banks (rows are 256 or 512 bytes). The former 2k swizzle paired them
// up: 2-way conflicts, measured as 28% of LDS cycles on the LM-head NN GEMM.
__device__ __forceinline__ int mnswz(int k) { return (4 * k) & 15; }

// Per-lane DMA offsets of one ROWS x BKT operand tile filled by NW waves.
template <int ROWS, int BKT, bool KMAJ, int NW>
struct Dma {
  static constexpr int CH = BKT / 8;
  static constexpr int INSTR = ROWS * BKT / 8 / 64 / NW;  // per wave per stage
  static_assert(INSTR >= 1 && INSTR * 64 * NW * 8 == ROWS * BKT, "a stage splits into whole DMA instructions");
  uint32_t voff[INSTR];  // bytes from the operand base for k0 = 0
  __device__ __forceinline__ void init(int row0, int64_t ld, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      if constexpr (KMAJ) {
        const int r = (i * NW + wave) * (64 / CH) + lane / CH;
        const int kc = (lane % CH) ^ kswz<CH>(r);
        voff[i] = (uint32_t)(((int64_t)(row0 + r) * ld + kc * 8) * 2);
      } else {
        constexpr int CPR = ROWS / 8, RPI = 64 / CPR;
        const int k = (i * NW + wave) * RPI + lane / CPR;
        const int c = (lane % CPR) ^ mnswz(k);
        voff[i] = (uint32_t)(((int64_t)k * ld + row0 + c * 8) * 2);
      }
    }
  }
  // issue the stage whose first k is k0 into the tile at `lds`
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rs, uint16_t* lds, int k0, int64_t ld, int wave) {
    const uint32_t soff = KMAJ ? (uint32_t)(k0 * 2) : (uint32_t)((int64_t)k0 * ld * 2);
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const int base_elems = (i * NW + wave) * 512;  // each instruction fills 64 x 16 bytes
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(lds + base_elems), 16, voff[i], soff, 0, 0);
    }
  }
};

// Masked register staging of one stage (used for a ragged K tail only).
template <int ROWS, int BKT, bool KMAJ, int NT>
__device__ __forceinline__ void stage_masked(const uint16_t* __restrict__ P, int64_t ld, int row0, int rows_lim,
                                             int k0, int k_lim, uint16_t* lds, int tid) {
  constexpr int CH = BKT / 8;
  constexpr int UNITS = ROWS * CH;  // 16-byte chunks
#pragma unroll
  for (int i = 0; i < (UNITS + NT - 1) / NT; ++i) {
    const int u = i * NT + tid;
    if (u >= UNITS) break;
    if constexpr (KMAJ) {
      const int r = u / CH, kc = u % CH;
      const int grow = row0 + r, gk = k0 + kc * 8;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (grow < rows_lim) v = load8(P + (int64_t)grow * ld + gk, k_lim - gk);
      *reinterpret_cast<u32x4*>(lds + r * BKT + ((kc ^ kswz<CH>(r)) << 3)) = v;
    } else {
      constexpr int CPR = ROWS / 8;
      const int k = u / CPR, c = u % CPR;
      const int gk = k0 + k, gm = row0 + c * 8;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (gk < k_lim) v = load8(P + (int64_t)gk * ld + gm, rows_lim - gm);
      *reinterpret_cast<u32x4*>(lds + k * ROWS + ((c ^ mnswz(k)) << 3)) = v;
    }
  }
}

// Fragment reader for a 32-row block of a tile: 8 bf16 of k = ks*16 + 8g .. +7.
template <int ROWS, int BKT, bool KMAJ>
struct Frag {
  static constexpr int CH = BKT / 8;
  int off[2];   // per-lane element offsets (K-major: row start; MN-major: two tr reads)
  int sw;       // K-major: row swizzle key
  __device__ __forceinline__ void init(int row, int lane) {
    if constexpr (KMAJ) {
      const int r = row + (lane & 31);
      off[0] = r * BKT;
      sw = kswz<CH>(r);
    } else {
      const int G = lane >> 4, j = lane & 15;
      const int g = G >> 1, h = G & 1;
      const int mn = row + 16 * h + 4 * (j & 3);
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int k = 8 * g + 4 * rr + (j >> 2);  // + ks*16 (does not change the swizzle key)
        off[rr] = k * ROWS + (((mn >> 3) ^ mnswz(k)) << 3) + (mn & 7);
      }
      sw = 0;
    }
  }
  __device__ __forceinline__ bf16x8 read(const uint16_t* tile, int ks, int lane) const {
    if constexpr (KMAJ) {
      const int kc = ks * 2 + (lane >> 5);
      return as_bf16x8(*reinterpret_cast<const u32x4*>(tile + off[0] + ((kc ^ sw) << 3)));
    } else {
      const uint16_t* t = tile + ks * 16 * ROWS;
      const u32x2 a = ds_read_tr16(t + off[0]), b = ds_read_tr16(t + off[1]);
      return as_bf16x8(u32x4{a[0], a[1], b[0], b[1]});
    }
  }
};


// Instruction order of one LDS stage for the scheduler: the first k16 step's R
// fragment reads, then each of the NM MFMAs of step ks followed by its share of
// step ks+1's reads, so LDS latency hides behind the MFMAs in flight (left to
// itself the compiler reuses one register set: read, wait, 4 MFMAs, read, ...).
template <int M, int NM, int R>
__device__ __forceinline__ void sched_ks() {
  if constexpr (M < NM) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    constexpr int lo = M * R / NM, hi = (M + 1) * R / NM;
    if constexpr (hi > lo) __builtin_amdgcn_sched_group_barrier(0x100, hi - lo, 0);  // ds_reads
    sched_ks<M + 1, NM, R>();
  }
}
template <int R, int NM, int KS, int KK = 0>
__device__ __forceinline__ void sched_stage() {
  if constexpr (KK == 0) __builtin_amdgcn_sched_group_barrier(0x100, R, 0);
  if constexpr (KK + 1 < KS) {
    sched_ks<0, NM, R>();
    sched_stage<R, NM, KS, KK + 1>();
  } else {
    __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
  }
}

// Merge (max, sum of 2^(x - max)) partials, both in log2 units; an empty
// partial is (-inf, 0).
__device__ __forceinline__ void ce_combine(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  s = s * fast_exp2(m - mn) + s2 * fast_exp2(m2 - mn);
  m = mn;
}

// wait until at most `later` stages (IPS DMA ops each) of this wave are outstanding
template <int IPS, int MAXL>
__device__ __forceinline__ void wait_stage(int later) {
  if constexpr (MAXL <= 0) {
    wait_vm<0>();
  } else {
    if (later >= MAXL) wait_vm<MAXL * IPS>();
    else wait_stage<IPS, MAXL - 1>(later);
  }
}

template <int BM, int BN, int BKT, int S, bool A_KMAJ, bool B_KMAJ, typename OutT, int EPI>
__global__ __launch_bounds__((BM * BN >= 65536) ? 512 : 256,
                             (BM * BN >= 65536) ? 1 : 2) void gemm2_kernel(GemmArgs g) {
  // 256 x 256 tiles run 8 waves (2 x 4), the others 4 (2 x 2); every wave
  // owns a WTM x 64 block of the tile.
  constexpr bool kHuge = BM * BN >= 65536;
  constexpr int NWV = kHuge ? 8 : 4;
  constexpr int NT = 64 * NWV;
  constexpr int WNW = BN / 64, WMW = NWV / WNW;
  static_assert(WNW * WMW == NWV, "wave layout");
  constexpr int WTM = BM / WMW, WTN = 64;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int STAGE = (BM + BN) * BKT;  // elements per stage
  // After the K loop the same LDS holds the epilogue: four 8 KB store slabs at
  // byte 0 and, from byte kExtra, the bias columns (1 KB) or the saved GELU
  // pre-activation tile (32 KB).
  constexpr bool kBias = EPI == NL_EPI_BIAS || EPI == NL_EPI_BIAS_GELU;
  constexpr bool kAux = EPI == NL_EPI_DGELU;
  static_assert(S == 2 || S == 3, "two or three pipeline stages");
  // Each pipeline stage is its own LDS object: the compiler can then prove that
  // the DMA filling one stage does not alias the reads of another and does not
  // make those reads wait for it.
  __shared__ __attribute__((aligned(16))) uint16_t st0[STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t st1[STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t st2[S > 2 ? STAGE : 8];
  // Epilogue LDS: four 8 KB store slabs (in the stage buffers), the bias
  // columns (1 KB) and, for the GELU backward, the saved pre-activation tile
  // (32 KB: the second stage buffer when stages are that large).
  constexpr bool kAuxInSt1 = kAux && STAGE * 2 >= BM * BN * 2;
  __shared__ __attribute__((aligned(16))) float sbias_lds[kBias ? 256 : 4];
  __shared__ __attribute__((aligned(16))) uint16_t aux_lds[kAux && !kAuxInSt1 ? BM * BN : 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WNW, wn = wave % WNW;

  int bid = blockIdx.x;
  {
    const int nwg = gridDim.x, per = nwg / 8;
    if (bid < per * 8) bid = (bid % 8) * per + bid / 8;
  }
  const int tiles_n = (g.N + BN - 1) / BN;
  const int tiles_m = (g.M + BM - 1) / BM;
  const int split = bid / g.tiles;
  const int tile = bid - split * g.tiles;
  constexpr int GM = 8;
  const int in_group = GM * tiles_n;
  const int first_m = (tile / in_group) * GM;
  const int gsize = min(tiles_m - first_m, GM);
  const int tm = first_m + (tile % in_group) % gsize;
  const int tn = (tile % in_group) / gsize;
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = split * g.k_chunk;
  const int kend = min(g.K, kbeg + g.k_chunk);
  const int nfull = kend > kbeg ? (kend - kbeg) / BKT : 0;
  const bool tail = kend > kbeg && ((kend - kbeg) % BKT) != 0;

  // Buffer descriptors clip at the end of each logical matrix, rounded up to
  // the 16-byte chunk that holds its last element: the range check zeroes
  // whole dwords, and an aligned chunk never crosses a page. The extra columns
  // only reach outputs that are not stored; a ragged K tail is staged with
  // element masks instead.
  const uint32_t a_bytes = (uint32_t)((((A_KMAJ ? (int64_t)(g.M - 1) * g.lda + g.K
                                                : (int64_t)(g.K - 1) * g.lda + g.M) * 2) + 15) & ~(int64_t)15);
  const uint32_t b_bytes = (uint32_t)((((B_KMAJ ? (int64_t)(g.N - 1) * g.ldb + g.K
                                                : (int64_t)(g.K - 1) * g.ldb + g.N) * 2) + 15) & ~(int64_t)15);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(g.A, a_bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(g.B, b_bytes);
  // The 8-wave TN tile (the LM-head weight gradient) gives each stage's DMA
  // to half of its waves, alternating by stage (waves w and w + 4 share a
  // SIMD). Issued by all 8 waves at once, the 64 instructions of a stage
  // queue in the CU's memory pipeline, and both waves of every SIMD sat in
  // the issue for 800+ cycles per stage with the MFMA pipe idle (the pipeline
  // itself moves the 64 KB in about 0.8 us: the stall is the burst, not the
  // bandwidth); this way one of the two computes meanwhile. Measured at
  // 512 x 50257 x 16384: 771-777 -> 737-744 us.
  // (Slower for the NT form, 672-695 -> 694-708 us, and for 128 x 128 tiles.)
  constexpr int DNW = (!A_KMAJ && !B_KMAJ && kHuge && S == 2) ? NWV / 2 : NWV;
  Dma<BM, BKT, A_KMAJ, DNW> da;
  Dma<BN, BKT, B_KMAJ, DNW> db;
  da.init(m0, g.lda, wave % DNW, lane);
  db.init(n0, g.ldb, wave % DNW, lane);
  constexpr int IPS = Dma<BM, BKT, A_KMAJ, DNW>::INSTR + Dma<BN, BKT, B_KMAJ, DNW>::INSTR;  // DMA ops per stage per issuing wave

  Frag<BM, BKT, A_KMAJ> fa[FM];
  Frag<BN, BKT, B_KMAJ> fb[FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) fa[i].init(wm * WTM + i * 32, lane);
#pragma unroll
  for (int j = 0; j < FN; ++j) fb[j].init(wn * WTN + j * 32, lane);

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  bf16x8 af[2][FM], bfr[2][FN];
  auto compute = [&](const uint16_t* sb) __attribute__((always_inline)) {
    const uint16_t* As = sb;
    const uint16_t* Bs = sb + BM * BKT;
#pragma unroll
    for (int i = 0; i < FM; ++i) af[0][i] = fa[i].read(As, 0, lane);
#pragma unroll
    for (int j = 0; j < FN; ++j) bfr[0][j] = fb[j].read(Bs, 0, lane);
#pragma unroll
    for (int ks = 0; ks < BKT / 16; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < BKT / 16) {
#pragma unroll
        for (int i = 0; i < FM; ++i) af[cur ^ 1][i] = fa[i].read(As, ks + 1, lane);
#pragma unroll
        for (int j = 0; j < FN; ++j) bfr[cur ^ 1][j] = fb[j].read(Bs, ks + 1, lane);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma32(bfr[cur][j], af[cur][i], acc[i][j]);
    }
    if constexpr (kHuge) {
      // ds_read instructions per k16 step: one per k-major fragment, two per transposed one
      constexpr int R = FM * (A_KMAJ ? 1 : 2) + FN * (B_KMAJ ? 1 : 2);
      sched_stage<R, FM * FN, BKT / 16>();
    }
  };
  auto issue = [&](uint16_t* sb, int st) __attribute__((always_inline)) {  // DMA of stage st (0-based in this split)
    if (DNW == NWV || wave / DNW == (st & 1)) {
      const int k0 = kbeg + st * BKT;
      da.issue(ra, sb, k0, g.lda, wave % DNW);
      db.issue(rb, sb + BM * BKT, k0, g.ldb, wave % DNW);
    }
  };

  // S-stage pipeline, unrolled by S so that every buffer is a fixed LDS object.
  // Step kt: wait until this wave's DMA of stage kt has landed (later stages
  // may stay in flight), barrier (stage kt complete for all waves, all waves
  // done with stage kt-1), start the DMA of stage kt+S-1 into the buffer of
  // stage kt-1, compute stage kt. With three stages the barrier is a bare
  // s_barrier (a memory clobber for the compiler): __syncthreads would also
  // wait for the DMA still in flight.
  auto step = [&](uint16_t* cur, uint16_t* nxt, int kt) __attribute__((always_inline)) {
    wait_stage<IPS, S - 2>(min(S - 2, nfull - 1 - kt));
    if constexpr (S == 2) __syncthreads();
    else asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // this wave's LDS reads done
    if (kt + S - 1 < nfull) issue(nxt, kt + S - 1);
    compute(cur);
  };
  if (nfull > 0) issue(st0, 0);
  if (S > 2 && nfull > 1) issue(st1, 1);
  if constexpr (S == 2) {
    for (int kt = 0; kt < nfull; kt += 2) {
      step(st0, st1, kt);
      if (kt + 1 >= nfull) break;
      step(st1, st0, kt + 1);
    }
  } else {
    for (int kt = 0; kt < nfull; kt += 3) {
      step(st0, st2, kt);
      if (kt + 1 >= nfull) break;
      step(st1, st0, kt + 1);
      if (kt + 2 >= nfull) break;
      step(st2, st1, kt + 2);
    }
  }
  if (tail) {
    __syncthreads();
    uint16_t* sb = (nfull % S) == 0 ? st0 : (nfull % S) == 1 ? st1 : st2;
    const int kt0 = kbeg + nfull * BKT;
    stage_masked<BM, BKT, A_KMAJ, NT>(g.A, g.lda, m0, g.M, kt0, kend, sb, tid);
    stage_masked<BN, BKT, B_KMAJ, NT>(g.B, g.ldb, n0, g.N, kt0, kend, sb + BM * BKT, tid);
    __syncthreads();
    compute(sb);
  }
  const int frow = lane & 31;
  const int g4 = (lane >> 5) * 4;
  if constexpr (EPI == kEpiCeStats) {
    // Lane (frow, g4) holds row frow of each 32-row block and 16 of every 32
    // columns; lanes l and l ^ 32 share a row. Per row: the wave's (max, sum)
    // over its WTN columns, then the WNW waves of a row band merged in LDS.
    // Logits are rounded in pairs (one v_cvt_pk_bf16_f32); column bounds are
    // checked only in the wave tile that crosses N, and the target's logit is
    // looked for only by lanes whose row's target lies in the wave tile.
    float s = g.alpha;
    if (g.alpha_dev) s *= *g.alpha_dev;
    static_assert(STAGE * 2 >= WNW * BM * 8, "row partials of all wave columns fit the first stage buffer");
    float2* red = reinterpret_cast<float2*>(st0);  // [WNW][BM]
    const int wc0 = n0 + wn * WTN;                  // first column of the wave tile
    const int nlim = g.N - wc0;                     // its valid columns (may be <= 0)
    const bool full = nlim >= WTN;
    __syncthreads();                                // every wave is done reading the stage buffers
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int ml = wm * WTM + i * 32 + frow;
      const int m = m0 + ml;
      const int tc = (m < g.M ? g.ce_tgt[m] - g.ce_v0 : -1) - wc0;
      uint32_t pk[FN][8];
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int h = 0; h < 8; ++h) pk[j][h] = pack_bf16x2(acc[i][j][2 * h] * s, acc[i][j][2 * h + 1] * s);
      // element 2h + b of pk[j] is column j*32 + (h >> 1)*8 + g4 + (h & 1)*2 + b
      auto col = [&](int j, int h, int b) { return j * 32 + (h >> 1) * 8 + g4 + (h & 1) * 2 + b; };
      float mx = -INFINITY;
      if (full) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int h = 0; h < 8; ++h) mx = fmaxf(mx, fmaxf(bf16_lo(pk[j][h]), bf16_hi(pk[j][h])));
      } else {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int h = 0; h < 8; ++h) {
            if (col(j, h, 0) < nlim) mx = fmaxf(mx, bf16_lo(pk[j][h]));
            if (col(j, h, 1) < nlim) mx = fmaxf(mx, bf16_hi(pk[j][h]));
          }
      }
      if ((unsigned)tc < (unsigned)WTN) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int h = 0; h < 8; ++h) {
            if (col(j, h, 0) == tc) g.ce_correct[m] = bf16_lo(pk[j][h]);
            if (col(j, h, 1) == tc) g.ce_correct[m] = bf16_hi(pk[j][h]);
          }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mx2 = mx * kLog2e;
      float sum = 0.f;
      if (full) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int h = 0; h < 8; ++h)
            sum += fast_exp2(__builtin_fmaf(bf16_lo(pk[j][h]), kLog2e, -mx2)) +
                   fast_exp2(__builtin_fmaf(bf16_hi(pk[j][h]), kLog2e, -mx2));
      } else {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int h = 0; h < 8; ++h) {
            if (col(j, h, 0) < nlim) sum += fast_exp2(__builtin_fmaf(bf16_lo(pk[j][h]), kLog2e, -mx2));
            if (col(j, h, 1) < nlim) sum += fast_exp2(__builtin_fmaf(bf16_hi(pk[j][h]), kLog2e, -mx2));
          }
      }
      sum += __shfl_xor(sum, 32, 64);
      if (lane < 32) red[wn * BM + ml] = make_float2(mx2, sum);
    }
    __syncthreads();
    for (int r = tid; r < BM; r += NT) {
      const int m = m0 + r;
      if (m >= g.M) break;
      float pm = -INFINITY, ps = 0.f;
#pragma unroll
      for (int w = 0; w < WNW; ++w) {
        const float2 v = red[w * BM + r];
        ce_combine(pm, ps, v.x, v.y);
      }
      reinterpret_cast<float2*>(g.ce_part)[(int64_t)m * tiles_n + tn] = make_float2(pm, ps);
    }
    return;
  }
  if (g.ws) {
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
          if (n < g.N)
            *reinterpret_cast<f32x4*>(W + (int64_t)m * g.ldw + n) =
                f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        }
    }
    return;
  }
  // Epilogue operands (bias columns, the saved pre-activation tile) are staged
  // into LDS by DMA before the first store: a wait on a vector load also waits
  // for every earlier store, so loads mixed into the store stream would
  // serialise it. The operand tiles' LDS is free once all waves pass the barrier.
  static_assert((!kBias && !kAux) || (BM == 128 && BN == 128), "the staged epilogue assumes 128 x 128 tiles");
  uint16_t* const xlds = kAuxInSt1 ? st1 : aux_lds;
  const float* sbias = sbias_lds;
  __syncthreads();
  if constexpr (kBias || kAux) {
    if constexpr (kBias) {
      // bias[n0 .. n0+255] -> 1 KB (only the first 128 are read); clipped at N
      if (wave == 0) {
        const __amdgpu_buffer_rsrc_t rbias = make_rsrc(g.bias, (uint32_t)g.N * 4u);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rbias, (lds_void*)sbias_lds, 16, (uint32_t)(n0 + lane * 4) * 4u, 0, 0,
                                                 0);
      }
    } else {
      // aux tile [128][128] bf16: row r at r*256 bytes, 16-byte chunk c at slot c ^ (r & 15)
      const uint32_t aux_bytes = (uint32_t)(((int64_t)g.M * g.ldaux) * 2);
      const __amdgpu_buffer_rsrc_t raux = make_rsrc(g.aux, aux_bytes);
#pragma unroll
      for (int i = 0; i < BM * BN * 2 / 1024 / NWV; ++i) {
        const int blk = i * NWV + wave;            // 1 KB block = 4 rows
        const int r = blk * 4 + (lane >> 4);
        const int c = (lane & 15) ^ (r & 15);
        const uint32_t off = (uint32_t)(((int64_t)(m0 + r) * g.ldaux + n0 + c * 8) * 2);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(raux, (lds_void*)(xlds + blk * 512), 16, off, 0, 0, 0);
      }
    }
    wait_vm<0>();
    __syncthreads();
  }
  float s = g.alpha;
  if (g.alpha_dev) s *= *g.alpha_dev;
  constexpr bool kCeGrad = EPI == kEpiCeGrad;
  if (!kCeGrad && g.beta != 0.f) {
    // C is read back: per-lane path (the reads sit between the stores)
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int ml = wm * WTM + i * 32 + frow;
      const int m = m0 + ml;
      if (m >= g.M) continue;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int nl = wn * WTN + j * 32 + q * 8 + g4;
          const int n = n0 + nl;
          if (n >= g.N) continue;
          float v[4] = {acc[i][j][4 * q + 0] * s, acc[i][j][4 * q + 1] * s, acc[i][j][4 * q + 2] * s,
                        acc[i][j][4 * q + 3] * s};
          f32x4 b = {0.f, 0.f, 0.f, 0.f};
          if constexpr (kBias) b = *reinterpret_cast<const f32x4*>(sbias + nl);
          epilogue_apply<OutT, EPI>(g, m, n, v, b, u32x2{0u, 0u});
        }
      }
    }
    return;
  }

  // Row-coalesced stores through LDS. A lane's MFMA results are 4-column
  // pieces of 32 different rows; storing them directly makes every store
  // instruction touch 32 rows. Instead each wave writes its 32-row slab (one
  // MFMA row block) into a private 8 KB LDS region, 16-byte chunks XOR-swizzled
  // by row, and reads it back so that consecutive lanes hold consecutive
  // 16-byte pieces of a row. Values are finished (scale, bias, GELU') group by
  // group on the way into LDS, which keeps few of them live in VGPRs.
  // A slab row holds the wave tile's WTN columns: CPR 16-byte chunks, chunk c
  // of row r at slot c ^ (r & (CPR - 1)).
  constexpr int SLAB = 32 * WTN * (int)sizeof(OutT);
  static_assert(STAGE * 2 >= NWV / 2 * SLAB, "a slab per wave in the first two stage buffers");
  static_assert(!kAuxInSt1 || NWV * SLAB <= STAGE * 2, "slabs and the aux tile share no bytes");
  uint8_t* wl = kAuxInSt1 ? reinterpret_cast<uint8_t*>(st0) + wave * SLAB
                          : reinterpret_cast<uint8_t*>(wave < NWV / 2 ? st0 : st1) + (wave % (NWV / 2)) * SLAB;
  // cross-entropy gradient: each lane's rows' lse (log2 units) and target column
  float ce_l2[FM];
  int ce_t[FM];
  float ce_gs = 0.f;
  if constexpr (kCeGrad) {
    ce_gs = g.ce_scale * (g.ce_scale_dev ? *g.ce_scale_dev : 1.f);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = m0 + wm * WTM + i * 32 + frow;
      ce_l2[i] = m < g.M ? g.ce_lse[m] * kLog2e : 0.f;
      ce_t[i] = m < g.M ? g.ce_tgt[m] - g.ce_v0 - n0 : -1;
    }
  }
  auto finish4 = [&](int i, int j, int q, float x[4]) {
    const int nl = wn * WTN + j * 32 + q * 8 + g4;
    f32x4 b = {0.f, 0.f, 0.f, 0.f};
    if constexpr (kBias) b = *reinterpret_cast<const f32x4*>(sbias + nl);
    u32x2 a = {0u, 0u};
    if constexpr (kAux) {
      const int ml = wm * WTM + i * 32 + frow;
      a = *reinterpret_cast<const u32x2*>(xlds + ml * 128 + (((nl >> 3) ^ (ml & 15)) << 3) + (nl & 7));
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = acc[i][j][4 * q + e] * s;
      if constexpr (kBias) x[e] += b[e];
      if constexpr (kAux) x[e] *= gelu_tanh_grad(e & 1 ? bf16_hi(a[e >> 1]) : bf16_lo(a[e >> 1]));
    }
    if constexpr (kCeGrad) {
      // the logits as bf16 (one packed conversion per pair), then the CE gradient
      const uint32_t p01 = pack_bf16x2(x[0], x[1]), p23 = pack_bf16x2(x[2], x[3]);
      const float l[4] = {bf16_lo(p01), bf16_hi(p01), bf16_lo(p23), bf16_hi(p23)};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p = fast_exp2(__builtin_fmaf(l[e], kLog2e, -ce_l2[i]));
        x[e] = (nl + e == ce_t[i] ? p - 1.f : p) * ce_gs;
      }
    }
  };
  // write the lane's 4 values of (slab row frow, columns j*32 + q*8 + g4 ..) into the slab
  auto at_bf16 = [&](int j, int q) {
    constexpr int CPR = WTN * 2 / 16;                   // WTN * 2-byte rows
    const int c = j * 32 + q * 8 + g4;
    return reinterpret_cast<u32x2*>(wl + frow * (WTN * 2) + ((((c * 2) >> 4) ^ (frow & (CPR - 1))) << 4) + ((c * 2) & 15));
  };
  auto put_bf16 = [&](int j, int q, const float x[4]) {
    *at_bf16(j, q) = u32x2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
  };
  auto put_f32 = [&](int j, int q, const float x[4]) {
    constexpr int CPR = WTN * 4 / 16;                   // WTN * 4-byte rows
    const int c = j * 32 + q * 8 + g4;
    *reinterpret_cast<f32x4*>(wl + frow * (WTN * 4) + ((((c * 4) >> 4) ^ (frow & (CPR - 1))) << 4)) =
        f32x4{x[0], x[1], x[2], x[3]};
  };
  // copy slab i (32 rows) from LDS to global rows, 16 bytes per lane
  auto copy_out = [&](auto tag, int i, void* base, int64_t ld) {
    using T = decltype(tag);
    constexpr int PITCH = WTN * (int)sizeof(T);
    constexpr int CPR = PITCH / 16;
    constexpr int EPC = 16 / (int)sizeof(T);
    constexpr int RPI = 64 / CPR;                       // slab rows per instruction
#pragma unroll
    for (int it = 0; it < 32 / RPI; ++it) {
      const int r = it * RPI + lane / CPR;
      const int ch = lane % CPR;
      const u32x4 val = *reinterpret_cast<const u32x4*>(wl + r * PITCH + ((ch ^ (r & (CPR - 1))) << 4));
      const int m = m0 + wm * WTM + i * 32 + r;
      const int n = n0 + wn * WTN + ch * EPC;
      if (m >= g.M || n >= g.N) continue;
      T* dst = reinterpret_cast<T*>(base) + (int64_t)m * ld + n;
      if (n + EPC <= g.N) {
        __builtin_nontemporal_store(val, reinterpret_cast<u32x4*>(dst));
      } else {
#pragma unroll
        for (int k = 0; k < EPC; ++k) {
          if (n + k >= g.N) break;
          if constexpr (sizeof(T) == 2) dst[k] = (T)(val[k >> 1] >> (16 * (k & 1)));
          else dst[k] = __uint_as_float(val[k]);
        }
      }
    }
  };
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    if constexpr (EPI == NL_EPI_BIAS_GELU) {
      // the pre-activation u = bf16(v + bias) goes to aux; C = gelu(u), with u
      // read back from the lane's own slab entries
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float x[4];
          finish4(i, j, q, x);
          put_bf16(j, q, x);
        }
      copy_out(uint16_t{}, i, g.aux, g.ldaux);
      u32x2 uu[FN][4];
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) uu[j][q] = *at_bf16(j, q);
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float x[4] = {gelu_tanh(bf16_lo(uu[j][q][0])), gelu_tanh(bf16_hi(uu[j][q][0])),
                              gelu_tanh(bf16_lo(uu[j][q][1])), gelu_tanh(bf16_hi(uu[j][q][1]))};
          if constexpr (sizeof(OutT) == 2) put_bf16(j, q, x);
          else put_f32(j, q, x);
        }
    } else {
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float x[4];
          finish4(i, j, q, x);
          if constexpr (sizeof(OutT) == 2) put_bf16(j, q, x);
          else put_f32(j, q, x);
        }
    }
    if constexpr (sizeof(OutT) == 2) copy_out(uint16_t{}, i, g.C, g.ldc);
    else copy_out(float{}, i, g.C, g.ldc);
  }
}

// ---------------------------------------------------------------------------
// Persistent kernel for short-K products without a split: 256 x 256 tiles
// for the LM-head forward (K = 512: 8 stages per tile, where a tile's
// first-stage load and its 128 KB store were 30% of its time), 128 x 128 tiles
// for smaller products with at least 4 tiles per workgroup, with no epilogue,
// the bias one or the bias + GELU one (u to aux, gelu(u) to C). Each workgroup
// (one per CU, or two with 128 x 128 tiles) walks its tiles in order. While a
// tile's last stage is computed, the next tile's first stage is already
// loading into the other buffer; the tile's stores then drain while the next
// tile computes. On gfx9 stores count in vmcnt, so the next
// tile's first wait is vmcnt(number of stores just issued): exact for interior
// tiles, whose store path has no bounds branches; after an edge tile it is
// vmcnt(0). Requires K % 128 == 0 (an even number of full stages, no tail).
// ---------------------------------------------------------------------------
template <bool A_KMAJ, bool B_KMAJ, typename OutT, int BM = 256, int BN = 256, int NWV = 8, int EPI = NL_EPI_NONE>
__global__ __launch_bounds__(NWV * 64, NWV == 8 ? 1 : 2) void gemm_persist_kernel(GemmArgs g) {
  static_assert(EPI == NL_EPI_NONE || EPI == NL_EPI_BIAS || EPI == NL_EPI_BIAS_GELU, "epilogues of the persistent kernel");
  static_assert(EPI != NL_EPI_BIAS_GELU || sizeof(OutT) == 2, "the GELU epilogue writes bf16");
  constexpr bool kBias = EPI != NL_EPI_NONE;
  // 256 x 256 tiles: 8 waves of 128 x 64, one workgroup per CU; 128 x 128
  // tiles: 4 waves of 64 x 64, two workgroups per CU
  constexpr int BKT = 64;
  constexpr int WNW = BN / 64, WMW = NWV / WNW, WTM = BM / WMW, WTN = 64, FM = WTM / 32, FN = WTN / 32;
  constexpr int STAGE = (BM + BN) * BKT;
  __shared__ __attribute__((aligned(16))) uint16_t st0[STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t st1[STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WNW, wn = wave % WNW;
  const int tiles_n = (g.N + BN - 1) / BN;
  const int tiles_m = (g.M + BM - 1) / BM;
  const int ntiles = tiles_m * tiles_n;
  // XCD x (= blockIdx.x % 8, how the hardware deals workgroups) owns the
  // contiguous logical tile range [x * per_x, (x + 1) * per_x); its workgroups
  // take every (gridDim.x / 8)-th tile of it, so each XCD's L2 sees neighbours.
  const int nx = gridDim.x / 8;
  const int xcd = blockIdx.x % 8, jj = blockIdx.x / 8;
  const int per_x = (ntiles + 7) / 8;
  const int t_end = min(ntiles, (xcd + 1) * per_x);
  constexpr int GM = 8;
  const int in_group = GM * tiles_n;
  auto decode = [&](int t, int& m0, int& n0) {
    const int first_m = (t / in_group) * GM;
    const int gsize = min(tiles_m - first_m, GM);
    m0 = (first_m + (t % in_group) % gsize) * BM;
    n0 = ((t % in_group) / gsize) * BN;
  };
  int t = xcd * per_x + jj;
  if (t >= t_end) return;
  const int nfull = g.K / BKT;  // even (K % 128 == 0)

  const uint32_t a_bytes = (uint32_t)((((A_KMAJ ? (int64_t)(g.M - 1) * g.lda + g.K
                                                : (int64_t)(g.K - 1) * g.lda + g.M) * 2) + 15) & ~(int64_t)15);
  const uint32_t b_bytes = (uint32_t)((((B_KMAJ ? (int64_t)(g.N - 1) * g.ldb + g.K
                                                : (int64_t)(g.K - 1) * g.ldb + g.N) * 2) + 15) & ~(int64_t)15);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(g.A, a_bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(g.B, b_bytes);
  Dma<BM, BKT, A_KMAJ, NWV> da;
  Dma<BN, BKT, B_KMAJ, NWV> db;
  Frag<BM, BKT, A_KMAJ> fa[FM];
  Frag<BN, BKT, B_KMAJ> fb[FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) fa[i].init(wm * WTM + i * 32, lane);
#pragma unroll
  for (int j = 0; j < FN; ++j) fb[j].init(wn * WTN + j * 32, lane);
  float s = g.alpha;
  if (g.alpha_dev) s *= *g.alpha_dev;

  f32x16 acc[FM][FN];
  bf16x8 af[2][FM], bfr[2][FN];
  auto compute = [&](const uint16_t* sb) __attribute__((always_inline)) {
    const uint16_t* As = sb;
    const uint16_t* Bs = sb + BM * BKT;
#pragma unroll
    for (int i = 0; i < FM; ++i) af[0][i] = fa[i].read(As, 0, lane);
#pragma unroll
    for (int j = 0; j < FN; ++j) bfr[0][j] = fb[j].read(Bs, 0, lane);
#pragma unroll
    for (int ks = 0; ks < BKT / 16; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < BKT / 16) {
#pragma unroll
        for (int i = 0; i < FM; ++i) af[cur ^ 1][i] = fa[i].read(As, ks + 1, lane);
#pragma unroll
        for (int j = 0; j < FN; ++j) bfr[cur ^ 1][j] = fb[j].read(Bs, ks + 1, lane);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma32(bfr[cur][j], af[cur][i], acc[i][j]);
    }
    constexpr int R = FM * (A_KMAJ ? 1 : 2) + FN * (B_KMAJ ? 1 : 2);
    sched_stage<R, FM * FN, BKT / 16>();
  };
  auto issue = [&](uint16_t* sb, int k0) {
    da.issue(ra, sb, k0, g.lda, wave);
    db.issue(rb, sb + BM * BKT, k0, g.ldb, wave);
  };
  // Raw barrier: the vector-memory waits before it are explicit (__syncthreads
  // would add vmcnt(0) and drain the previous tile's stores). It waits for this
  // wave's LDS reads itself: the compiler may place the MFMAs that consume a
  // stage's last fragment reads after the barrier, and another wave's DMA into
  // that stage buffer, issued right after it, could then overwrite fragments
  // still being read. (Found as wrong output tiles of this kernel when an
  // in-place CE kernel ran beside it on another stream.)
  auto barrier = [&]() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  constexpr int PITCH = 64 * (int)sizeof(OutT);  // one 32 x 64 slab per wave and store round
  constexpr int CPR = PITCH / 16;
  constexpr int EPC = 16 / (int)sizeof(OutT);
  constexpr int RPI = 64 / CPR;
  // store instructions per wave, interior tile (the GELU epilogue stores u and gelu(u))
  constexpr int kStores = FM * (32 / RPI) * (EPI == NL_EPI_BIAS_GELU ? 2 : 1);
  static_assert(NWV * 32 * PITCH <= STAGE * 2, "slabs fit one stage buffer");
  static_assert(kStores < 64, "vmcnt range");
  // the bias of the lane's columns wn*WTN + j*32 + q*8 + g4 + 0..3, loaded at
  // the start of each tile (complete before its epilogue: later waits cover it)
  f32x4 bias_r[kBias ? FN : 1][4];
  auto load_bias = [&](int nb) {
    if constexpr (kBias) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = nb + wn * WTN + j * 32 + q * 8 + ((lane >> 5) * 4);
          if (n + 4 <= g.N) {
            bias_r[j][q] = *reinterpret_cast<const f32x4*>(g.bias + n);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) bias_r[j][q][e] = n + e < g.N ? g.bias[n + e] : 0.f;
          }
        }
    }
  };
  const int frow = lane & 31;
  const int g4 = (lane >> 5) * 4;
  uint8_t* wl = reinterpret_cast<uint8_t*>(st1) + wave * (32 * PITCH);

  int m0, n0;
  decode(t, m0, n0);
  da.init(m0, g.lda, wave, lane);
  db.init(n0, g.ldb, wave, lane);
  issue(st0, 0);
  bool pend_stores = false;  // interior stores of the previous tile still in flight
  while (true) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    const int t_next = t + nx;
    const bool has_next = t_next < t_end;
    int m1 = 0, n1 = 0;
    for (int kt = 0; kt < nfull; kt += 2) {
      if (kt == 0 && pend_stores) wait_vm<kStores>();
      else wait_vm<0>();
      barrier();
      if (kt == 0) load_bias(n0);
      issue(st1, kt * BKT + BKT);
      compute(st0);
      wait_vm<0>();
      barrier();
      if (kt + 2 < nfull) {
        issue(st0, (kt + 2) * BKT);
      } else if (has_next) {
        decode(t_next, m1, n1);
        da.init(m1, g.lda, wave, lane);
        db.init(n1, g.ldb, wave, lane);
        issue(st0, 0);
      }
      compute(st1);
    }
    // epilogue: every wave done with st1 -> slabs there; st0 holds the next
    // tile's first stage (in flight)
    __builtin_amdgcn_s_waitcnt((63 & 15) | ((63 >> 4) << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
    barrier();
    const bool interior = m0 + BM <= g.M && n0 + BN <= g.N;
    // slab row r, 16-byte chunk ch -> rows of the output at base (ld)
    auto copy_slab = [&](int i, auto tag, void* base, int64_t ld) __attribute__((always_inline)) {
      using T = decltype(tag);
      constexpr int P = 64 * (int)sizeof(T), CP = P / 16, EC = 16 / (int)sizeof(T), RI = 64 / CP;
#pragma unroll
      for (int it = 0; it < 32 / RI; ++it) {
        const int r = it * RI + lane / CP;
        const int ch = lane % CP;
        const u32x4 val = *reinterpret_cast<const u32x4*>(wl + r * P + ((ch ^ (r & (CP - 1))) << 4));
        const int mm = m0 + wm * WTM + i * 32 + r;
        const int n = n0 + wn * WTN + ch * EC;
        T* dst = reinterpret_cast<T*>(base) + (int64_t)mm * ld + n;
        if (interior) {
          __builtin_nontemporal_store(val, reinterpret_cast<u32x4*>(dst));
        } else {
          if (mm >= g.M || n >= g.N) continue;
          if (n + EC <= g.N) {
            __builtin_nontemporal_store(val, reinterpret_cast<u32x4*>(dst));
          } else {
#pragma unroll
            for (int k = 0; k < EC; ++k) {
              if (n + k >= g.N) break;
              if constexpr (sizeof(T) == 2) dst[k] = (T)(val[k >> 1] >> (16 * (k & 1)));
              else dst[k] = __uint_as_float(val[k]);
            }
          }
        }
      }
    };
    auto slab_bf16 = [&](int j, int q) {
      const int c = j * 32 + q * 8 + g4;
      return reinterpret_cast<u32x2*>(wl + frow * 128 + ((((c * 2) >> 4) ^ (frow & 7)) << 4) + ((c * 2) & 15));
    };
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float x[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x[e] = acc[i][j][4 * q + e] * s;
            if constexpr (kBias) x[e] += bias_r[j][q][e];
          }
          const int c = j * 32 + q * 8 + g4;
          if constexpr (sizeof(OutT) == 2) {
            *slab_bf16(j, q) = u32x2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
          } else {
            *reinterpret_cast<f32x4*>(wl + frow * 256 + ((((c * 4) >> 4) ^ (frow & 15)) << 4)) =
                f32x4{x[0], x[1], x[2], x[3]};
          }
        }
      if constexpr (EPI == NL_EPI_BIAS_GELU) {
        // the pre-activation u = bf16(v + bias) goes to aux; then C = gelu(u)
        // from the lane's own slab entries
        copy_slab(i, uint16_t{}, g.aux, g.ldaux);
        u32x2 uu[FN][4];
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) uu[j][q] = *slab_bf16(j, q);
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *slab_bf16(j, q) = u32x2{pack_bf16x2(gelu_tanh(bf16_lo(uu[j][q][0])), gelu_tanh(bf16_hi(uu[j][q][0]))),
                                     pack_bf16x2(gelu_tanh(bf16_lo(uu[j][q][1])), gelu_tanh(bf16_hi(uu[j][q][1])))};
      }
      copy_slab(i, OutT{}, g.C, g.ldc);
    }
    if (!has_next) break;
    pend_stores = interior;
    t = t_next;
    m0 = m1;
    n0 = n1;
  }
}

// Explicit instantiations: every (layout, output, epilogue) combination the
// dispatcher can launch gets its host stub emitted.
#define NL_I(AK, BKM, T, E) template __global__ void gemm2_kernel<128, 128, 64, 2, AK, BKM, T, E>(GemmArgs);
#define NL_I4(T, E) NL_I(true, false, T, E) NL_I(true, true, T, E) NL_I(false, false, T, E) NL_I(false, true, T, E)
#define NL_I8(E) NL_I4(float, E) NL_I4(uint16_t, E)
NL_I8(NL_EPI_NONE)
NL_I8(NL_EPI_BIAS)
NL_I8(NL_EPI_BIAS_GELU)
NL_I8(NL_EPI_DGELU)
template __global__ void gemm2_kernel<256, 128, 32, 2, true, false, float, NL_EPI_NONE>(GemmArgs);
template __global__ void gemm2_kernel<256, 256, 64, 2, true, false, uint16_t, kEpiCeStats>(GemmArgs);
template __global__ void gemm2_kernel<256, 256, 64, 2, true, false, uint16_t, kEpiCeGrad>(GemmArgs);
template __global__ void gemm2_kernel<256, 256, 64, 2, true, true, float, NL_EPI_NONE>(GemmArgs);
template __global__ void gemm_persist_kernel<true, true, float>(GemmArgs);
template __global__ void gemm_persist_kernel<true, true, uint16_t>(GemmArgs);
template __global__ void gemm_persist_kernel<true, false, float>(GemmArgs);
template __global__ void gemm_persist_kernel<true, false, uint16_t>(GemmArgs);
template __global__ void gemm_persist_kernel<false, false, float>(GemmArgs);
template __global__ void gemm_persist_kernel<false, false, uint16_t>(GemmArgs);
template __global__ void gemm_persist_kernel<true, false, float, 128, 128, 4>(GemmArgs);
template __global__ void gemm_persist_kernel<true, false, uint16_t, 128, 128, 4>(GemmArgs);
template __global__ void gemm_persist_kernel<true, true, float, 128, 128, 4>(GemmArgs);
template __global__ void gemm_persist_kernel<true, true, uint16_t, 128, 128, 4>(GemmArgs);
template __global__ void gemm_persist_kernel<true, false, float, 128, 128, 4, NL_EPI_BIAS>(GemmArgs);
template __global__ void gemm_persist_kernel<true, false, uint16_t, 128, 128, 4, NL_EPI_BIAS>(GemmArgs);
template __global__ void gemm_persist_kernel<true, true, float, 128, 128, 4, NL_EPI_BIAS>(GemmArgs);
template __global__ void gemm_persist_kernel<true, true, uint16_t, 128, 128, 4, NL_EPI_BIAS>(GemmArgs);
template __global__ void gemm_persist_kernel<true, false, uint16_t, 128, 128, 4, NL_EPI_BIAS_GELU>(GemmArgs);
template __global__ void gemm_persist_kernel<true, true, uint16_t, 128, 128, 4, NL_EPI_BIAS_GELU>(GemmArgs);
template __global__ void gemm2_kernel<256, 256, 64, 2, true, true, uint16_t, NL_EPI_NONE>(GemmArgs);
template __global__ void gemm2_kernel<256, 256, 64, 2, true, false, float, NL_EPI_NONE>(GemmArgs);
template __global__ void gemm2_kernel<256, 256, 64, 2, true, false, uint16_t, NL_EPI_NONE>(GemmArgs);
template __global__ void gemm2_kernel<256, 256, 64, 2, false, false, float, NL_EPI_NONE>(GemmArgs);
template __global__ void gemm2_kernel<256, 256, 64, 2, false, false, uint16_t, NL_EPI_NONE>(GemmArgs);
template __global__ void gemm2_kernel<256, 128, 32, 2, true, false, uint16_t, NL_EPI_NONE>(GemmArgs);
template __global__ void gemm2_kernel<256, 128, 32, 2, false, false, float, NL_EPI_NONE>(GemmArgs);
template __global__ void gemm2_kernel<256, 128, 32, 2, false, false, uint16_t, NL_EPI_NONE>(GemmArgs);
#undef NL_I8
#undef NL_I4
#undef NL_I

// beta*C for the degenerate K == 0 case is handled by the main kernel (nk = 0).

// C = epilogue(alpha * s * sum_split ws[split]), summed in split order (deterministic).
// Block = 64 column groups of 4 x 4 rows; grid (ceil(N/256), min(ceil(M/4), 65535)),
// rows strided by the grid. The partials of one group are loaded 8 splits at a
// time with every load in flight before the first add (the adds stay in split
// order), so a thread waits for one memory latency per 8 splits, not per split.
template <typename OutT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs g, int splits) {
  const int n = ((int)blockIdx.x * 64 + ((int)threadIdx.x & 63)) * 4;
  if (n >= g.N) return;
  float s = g.alpha;
  if (g.alpha_dev) s *= *g.alpha_dev;
  const int64_t plane = (int64_t)g.M * g.ldw;
  for (int64_t m = (int64_t)blockIdx.y * 4 + ((int)threadIdx.x >> 6); m < g.M; m += (int64_t)gridDim.y * 4) {
    const float* w = g.ws + m * g.ldw + n;
    f32x4 acc = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(w));
    int sp = 1;
    for (; sp + 8 <= splits; sp += 8) {
      f32x4 p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) p[j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(w + (sp + j) * plane));
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc[0] += p[j][0];
        acc[1] += p[j][1];
        acc[2] += p[j][2];
        acc[3] += p[j][3];
      }
    }
    for (; sp < splits; ++sp) {
      const f32x4 p = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(w + sp * plane));
      acc[0] += p[0];
      acc[1] += p[1];
      acc[2] += p[2];
      acc[3] += p[3];
    }
    float v[4] = {acc[0] * s, acc[1] * s, acc[2] * s, acc[3] * s};
    epilogue4_any<OutT>(g, m, n, v);
  }
}

// Tile configuration and K split of one product (shared by the workspace query).
// Compute units of the current device (cached per device).
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

struct Plan {
  int big;     // 1: 256 x 128 tiles (the very large products), 0: 128 x 128
  int tiles;
  int splits;
  int k_chunk;
  int64_t ldw;
  size_t ws_bytes;
};

Plan make_plan(int opA, int opB, int M, int N, int K, int epi) {
  Plan p;
  p.big = 0;
  p.tiles = (int)((int64_t)((M + 127) / 128) * ((N + 127) / 128));
  p.splits = 1;
  p.k_chunk = K > 0 ? K : 1;
  // skinny outputs with a long reduction (weight gradients, K = tokens): split K.
  // X^T dY (TN) products: a power-of-two split towards 512 workgroups, >= 1024 k
  // per split (measured on MI355X at the model's weight-gradient shapes: 10-20%
  // faster than the generic rule below); others: ~640 workgroups, >= 512 k.
  if (opA == NL_OP_T && opB == NL_OP_N && p.tiles < 256 && K >= 2048) {
    int want = 1;
    while (want * 2 * p.tiles <= 512) want *= 2;
    const int sp = want < K / 1024 ? want : K / 1024;
    if (sp > 1) {
      int chunk = (K + sp - 1) / sp;
      chunk = (chunk + BK - 1) / BK * BK;
      p.k_chunk = chunk;
      p.splits = (K + chunk - 1) / chunk;
    }
  } else if ((p.tiles < 256 && K >= 1024) || (p.tiles < 1024 && K >= 16384)) {
    int want = (p.tiles < 256 ? 640 + p.tiles - 1 : 1024 + p.tiles - 1) / p.tiles;
    int maxs = K / 512;
    int sp = want < maxs ? want : maxs;
    if (sp > 1) {
      int chunk = (K + sp - 1) / sp;
      chunk = (chunk + BK - 1) / BK * BK;
      p.k_chunk = chunk;
      p.splits = (K + chunk - 1) / chunk;
    }
  }
  // 256 x 128 tiles (4 waves of 128 x 64) for the largest products whose B is
  // k-by-n (NN, TN) and that need no fused epilogue: measured on MI355X, they
  // beat 128 x 128 on the LM head (TN 16384-deep: ~15%), lose on the FFN sizes.
  if (p.splits == 1 && opB == NL_OP_N && epi == NL_EPI_NONE &&
      ((opA == NL_OP_T && p.tiles >= 1024) || (opA == NL_OP_N && p.tiles >= 8192))) {
    p.big = 1;
    p.tiles = (int)((int64_t)((M + 255) / 256) * ((N + 127) / 128));
  }
  // 256 x 256 tiles (8 waves of 128 x 64, 64-k stages) for products of
  // >= 100 GFLOP without a fused epilogue (the LM head). Each CU then moves
  // half the operand bytes, and issues half the DMA instructions and barriers,
  // per flop of a 128 x 128 tile. Measured at the LM-head shapes: NN 1076 ->
  // 896 us, NT 1186 -> 897 us, TN 931 -> 811 us.
  // One workgroup per CU, so a short grid splits K up to 256 workgroups.
  if (epi == NL_EPI_NONE && !(opA == NL_OP_T && opB == NL_OP_T) && 2.0 * M * N * K >= 1e11) {
    p.big = 2;
    p.tiles = (int)((int64_t)((M + 255) / 256) * ((N + 255) / 256));
    p.splits = 1;
    p.k_chunk = K;
    if (p.tiles < 256 && K >= 4096) {
      const int sp = 256 / p.tiles;
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

// Launch one product whose operands fit 32-bit buffer offsets (the caller,
// run_product, splits anything larger).
template <bool AK, bool BK_, typename OutT>
void launch_cfg(GemmArgs g, const Plan& p, hipStream_t st) {
  g.tiles = p.tiles;
  g.k_chunk = p.k_chunk;
  // Pipeline: two 64-k stages for every layout. For NN, 32-k stages (half the
  // LDS, more workgroups per CU) are within a few percent when the operands
  // sit in the last-level cache, but an operand that the previous kernel has
  // just written comes from DRAM, and 64-byte row pieces read it a third
  // slower than 128-byte ones (FFN-down 16384 x 512 x 2048 on a cold input:
  // 66 -> 58 us; in the training step 52-59 -> 42-47 us).
  auto launch2 = [&](int grid) {
    if constexpr (AK || !BK_) {
      if (p.big == 2) {
        // short-K products without a split: one persistent workgroup per CU
        if (!g.ws && g.beta == 0.f && g.K % 128 == 0 && g.K <= 4096) {
          const int cus = cu_count();
          const int ntiles = (int)((int64_t)((g.M + 255) / 256) * ((g.N + 255) / 256));
          const int G = std::max(8, std::min(cus / 8 * 8, (ntiles + 7) / 8 * 8));
          hipLaunchKernelGGL((gemm_persist_kernel<AK, BK_, OutT>), dim3(G), dim3(512), 0, st, g);
          return;
        }
        hipLaunchKernelGGL((gemm2_kernel<256, 256, 64, 2, AK, BK_, OutT, NL_EPI_NONE>), dim3(grid), dim3(512), 0, st, g);
        return;
      }
    }
    if constexpr (!BK_) {
      if (p.big == 1) {
        hipLaunchKernelGGL((gemm2_kernel<256, 128, 32, 2, AK, BK_, OutT, NL_EPI_NONE>), dim3(grid), dim3(256), 0, st, g);
        return;
      }
    }
    constexpr int BKT = 64, NS = 2;
    // Short-K products with at least 4 tiles per workgroup and no epilogue or a
    // bias / bias + GELU one (QKV and FFN-up): the persistent kernel, two
    // 128 x 128 workgroups per CU, each loading its next tile's first stage
    // under its current tile's last one and storing a tile while computing the
    // next. Measured at 16384 x 1536 x 512: 37 -> 34 us (operands in the
    // caches), 42 -> 40 us (flushed first).
    if constexpr (AK) {
      const bool epi_ok = g.epi == NL_EPI_NONE || g.epi == NL_EPI_BIAS ||
                          (g.epi == NL_EPI_BIAS_GELU && sizeof(OutT) == 2);
      // (K = 0 stays on gemm2_kernel, which issues no DMA then: A and B may be null)
      if (!g.ws && g.beta == 0.f && epi_ok && g.K >= 128 && g.K % 128 == 0 && g.K <= 4096) {
        const int cus = cu_count();
        const int ntiles = (int)((int64_t)((g.M + 127) / 128) * ((g.N + 127) / 128));
        if (ntiles >= 4 * cus) {
          const dim3 grid(std::max(8, cus * 2 / 8 * 8)), block(256);
          if (g.epi == NL_EPI_BIAS) {
            hipLaunchKernelGGL((gemm_persist_kernel<AK, BK_, OutT, 128, 128, 4, NL_EPI_BIAS>), grid, block, 0, st, g);
          } else if (g.epi == NL_EPI_BIAS_GELU) {
            if constexpr (sizeof(OutT) == 2)
              hipLaunchKernelGGL((gemm_persist_kernel<AK, BK_, OutT, 128, 128, 4, NL_EPI_BIAS_GELU>), grid, block, 0,
                                 st, g);
          } else {
            hipLaunchKernelGGL((gemm_persist_kernel<AK, BK_, OutT, 128, 128, 4>), grid, block, 0, st, g);
          }
          return;
        }
      }
    }
    // with split K the epilogue runs in the reduction kernel
    const int epi = g.ws ? NL_EPI_NONE : g.epi;
    switch (epi) {
      case NL_EPI_BIAS:
        hipLaunchKernelGGL((gemm2_kernel<128, 128, BKT, NS, AK, BK_, OutT, NL_EPI_BIAS>), dim3(grid), dim3(256), 0, st, g);
        break;
      case NL_EPI_BIAS_GELU:
        hipLaunchKernelGGL((gemm2_kernel<128, 128, BKT, NS, AK, BK_, OutT, NL_EPI_BIAS_GELU>), dim3(grid), dim3(256), 0,
                           st, g);
        break;
      case NL_EPI_DGELU:
        hipLaunchKernelGGL((gemm2_kernel<128, 128, BKT, NS, AK, BK_, OutT, NL_EPI_DGELU>), dim3(grid), dim3(256), 0, st,
                           g);
        break;
      default:
        hipLaunchKernelGGL((gemm2_kernel<128, 128, BKT, NS, AK, BK_, OutT, NL_EPI_NONE>), dim3(grid), dim3(256), 0, st, g);
    }
  };
  if (p.splits > 1) {
    g.ldw = p.ldw;  // g.ws already set by the caller
    launch2(p.tiles * p.splits);
    const dim3 grid((unsigned)((g.N + 255) / 256), (unsigned)std::min<int64_t>(((int64_t)g.M + 3) / 4, 65535));
    hipLaunchKernelGGL((splitk_reduce_kernel<OutT>), grid, dim3(256), 0, st, g, p.splits);
  } else {
    g.ws = nullptr;
    launch2(p.tiles);
  }
}

template <typename OutT>
void launch_typed(int opA, int opB, const GemmArgs& g, const Plan& p, hipStream_t st) {
  // A is k-major when not transposed; B is k-major when transposed.
  if (opA == NL_OP_N && opB == NL_OP_N) launch_cfg<true, false, OutT>(g, p, st);
  else if (opA == NL_OP_N && opB == NL_OP_T) launch_cfg<true, true, OutT>(g, p, st);
  else if (opA == NL_OP_T && opB == NL_OP_N) launch_cfg<false, false, OutT>(g, p, st);
  else launch_cfg<false, true, OutT>(g, p, st);
}

// ---------------------------------------------------------------------------
// Products beyond the reach of 32-bit buffer offsets
// ---------------------------------------------------------------------------
// The kernels address each operand (and the DGELU aux) through a buffer
// descriptor with 32-bit byte offsets, reading up to one tile past the end
// (the range check zeroes those rows). A product whose operand extent reaches
// 2 GB is cut into sub-products that each fit, run in order on the stream:
//   * a k-contiguous A (or the aux) too long in M: panels of rows of C;
//   * a k-contiguous B too long in N: panels of columns of C;
//   * a k-strided A or B (stored [K][ld]) too long in K: chunks of K, the
//     later chunks added into C with beta = 1 (fp32 C, no GELU epilogue;
//     a bias is added by the first chunk only).
// Panels are balanced and rounded to whole 256-row tiles; K chunks to 64.
constexpr int64_t kOffsetLimit = (int64_t)1 << 31;

// rows per panel so that (rows + slack) * row_bytes stays below 2 GB, for a
// dimension of `total` rows cut into as few balanced panels as possible
int64_t panel_rows(int64_t total, int64_t row_bytes, int64_t slack, int64_t quantum) {
  int64_t cap = kOffsetLimit / row_bytes - slack - 1;
  cap = cap / quantum * quantum;
  if (cap < quantum) return 0;
  const int64_t panels = (total + cap - 1) / cap;
  int64_t per = (total + panels - 1) / panels;
  return (per + quantum - 1) / quantum * quantum;
}

// Calls f(sub) for every sub-product of g in launch order; f returns a status.
template <class F>
int for_each_subproduct(int opA, int opB, const GemmArgs& g, int c_dtype, F&& f) {
  const bool AK = opA == NL_OP_N, BKM = opB == NL_OP_T;
  const int64_t esz = c_dtype == NL_DTYPE_F32 ? 4 : 2;
  const int64_t aux_ld = g.epi == NL_EPI_DGELU ? g.ldaux : 0;
  const int64_t m_row_bytes = std::max<int64_t>(AK ? g.lda * 2 : 0, aux_ld * 2);
  if (g.M > 256 && m_row_bytes > 0 && ((int64_t)g.M + 256) * m_row_bytes >= kOffsetLimit) {
    const int64_t per = panel_rows(g.M, m_row_bytes, 256, 256);
    if (per == 0) return nl_set_error(NL_EUNSUPPORTED, "gemm: one 256-row panel of A spans 2 GB");
    for (int64_t m0 = 0; m0 < g.M; m0 += per) {
      GemmArgs s = g;
      s.M = (int)std::min<int64_t>(per, g.M - m0);
      s.A = AK ? g.A + m0 * g.lda : g.A + m0;
      s.C = static_cast<char*>(g.C) + m0 * g.ldc * esz;
      if (g.aux) s.aux = g.aux + m0 * g.ldaux;
      int rc = for_each_subproduct(opA, opB, s, c_dtype, f);
      if (rc) return rc;
    }
    return NL_OK;
  }
  if (BKM && g.N > 256 && ((int64_t)g.N + 256) * g.ldb * 2 >= kOffsetLimit) {
    const int64_t per = panel_rows(g.N, g.ldb * 2, 256, 256);
    if (per == 0) return nl_set_error(NL_EUNSUPPORTED, "gemm: one 256-row panel of B spans 2 GB");
    for (int64_t n0 = 0; n0 < g.N; n0 += per) {
      GemmArgs s = g;
      s.N = (int)std::min<int64_t>(per, g.N - n0);
      s.B = g.B + n0 * g.ldb;
      s.C = static_cast<char*>(g.C) + n0 * esz;
      if (g.bias) s.bias = g.bias + n0;
      if (g.aux) s.aux = g.aux + n0;
      int rc = for_each_subproduct(opA, opB, s, c_dtype, f);
      if (rc) return rc;
    }
    return NL_OK;
  }
  const int64_t k_row_bytes = std::max<int64_t>(AK ? 0 : g.lda * 2, BKM ? 0 : g.ldb * 2);
  if (g.K > BK && k_row_bytes > 0 && ((int64_t)g.K + BK) * k_row_bytes >= kOffsetLimit) {
    if (c_dtype != NL_DTYPE_F32 || (g.epi != NL_EPI_NONE && g.epi != NL_EPI_BIAS))
      return nl_set_error(NL_EUNSUPPORTED,
                          "gemm: a k-strided operand spanning 2 GB needs an fp32 C and no GELU epilogue");
    const int64_t per = panel_rows(g.K, k_row_bytes, BK, BK);
    if (per == 0) return nl_set_error(NL_EUNSUPPORTED, "gemm: 64 rows of a k-strided operand span 2 GB");
    for (int64_t k0 = 0; k0 < g.K; k0 += per) {
      GemmArgs s = g;
      s.K = (int)std::min<int64_t>(per, g.K - k0);
      s.A = AK ? g.A + k0 : g.A + k0 * g.lda;
      s.B = BKM ? g.B + k0 : g.B + k0 * g.ldb;
      if (k0 > 0) {
        s.beta = 1.f;
        s.epi = NL_EPI_NONE;
        s.bias = nullptr;
      }
      int rc = for_each_subproduct(opA, opB, s, c_dtype, f);
      if (rc) return rc;
    }
    return NL_OK;
  }
  // what is left must fit (a single tile's rows may still be too wide)
  const int64_t a_ext = (AK ? (int64_t)g.M + 256 : (int64_t)g.K + BK) * g.lda * 2;
  const int64_t b_ext = (BKM ? (int64_t)g.N + 256 : (int64_t)g.K + BK) * g.ldb * 2;
  const int64_t x_ext = ((int64_t)g.M + 256) * aux_ld * 2;
  if (a_ext >= kOffsetLimit || b_ext >= kOffsetLimit || x_ext >= kOffsetLimit)
    return nl_set_error(NL_EUNSUPPORTED, "gemm: rows of an operand too long for 32-bit buffer offsets");
  return f(g);
}

// ---------------------------------------------------------------------------
// Fused LM head + cross-entropy (linear_cross_entropy)
// ---------------------------------------------------------------------------

constexpr int kLceTile = 256;  // the 256 x 256 tiles of the LM-head GEMM

int lce_tiles_n(int V) { return (V + kLceTile - 1) / kLceTile; }

// Per row: merge the tiles' (max, sum) partials into lse; loss = lse - the
// target's logit (NaN for a target outside [0, V)). One wave per row.
__global__ __launch_bounds__(256) void lce_merge_kernel(int M, int V, int tiles_n, const float2* __restrict__ part,
                                                        const float* __restrict__ correct,
                                                        const int32_t* __restrict__ tgt, float* __restrict__ loss,
                                                        float* __restrict__ lse) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  float pm = -INFINITY, ps = 0.f;
  for (int k = lane; k < tiles_n; k += 64) {
    const float2 v = part[(int64_t)row * tiles_n + k];
    ce_combine(pm, ps, v.x, v.y);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(pm, o, 64), s2 = __shfl_xor(ps, o, 64);
    ce_combine(pm, ps, m2, s2);
  }
  if (lane == 0) {
    const float l = (pm + fast_log2(ps)) * kLn2;
    const int t = tgt[row];
    lse[row] = l;
    loss[row] = (t >= 0 && t < V) ? l - correct[row] : __builtin_nanf("");
  }
}

// One launch of the 256 x 256 NN kernel over X[M][D] . W[D][vn] with a CE epilogue.
template <int EPI>
void launch_lce(GemmArgs g, hipStream_t st) {
  g.tiles = (int)((int64_t)((g.M + kLceTile - 1) / kLceTile) * lce_tiles_n(g.N));
  g.k_chunk = g.K;
  g.ws = nullptr;
  hipLaunchKernelGGL((gemm2_kernel<kLceTile, kLceTile, 64, 2, true, false, uint16_t, EPI>), dim3(g.tiles), dim3(512),
                     0, st, g);
}

int check_lce_args(int M, int D, int V, const void* X, int64_t ldx, const void* W, int64_t ldw, const void* tgt) {
  if (M < 0 || D <= 0 || V <= 0) return nl_set_error(NL_EINVAL, "lce: need M >= 0, D > 0, V > 0");
  if (M > 0 && (!X || !W || !tgt)) return nl_set_error(NL_EINVAL, "lce: null pointer");
  if (ldx < D || ldw < V) return nl_set_error(NL_EINVAL, "lce: leading dimension too small");
  if ((((uintptr_t)X | (uintptr_t)W) & 15) != 0 || ((ldx | ldw) & 7) != 0)
    return nl_set_error(NL_EALIGN, "lce: X and W 16-byte aligned, ldx and ldw multiples of 8");
  // the kernel addresses X and W with 32-bit buffer offsets (up to a tile past the end)
  if (((int64_t)M + kLceTile) * ldx * 2 >= ((int64_t)1 << 31) || ((int64_t)D + 64) * ldw * 2 >= ((int64_t)1 << 31))
    return nl_set_error(NL_EUNSUPPORTED, "lce: X or W larger than 2 GiB");
  return NL_OK;
}

GemmArgs lce_args(int M, int D, int N, const nl_bf16* X, int64_t ldx, const nl_bf16* W, int64_t ldw,
                  const int32_t* tgt, int v0) {
  GemmArgs g{};
  g.M = M;
  g.N = N;
  g.K = D;
  g.A = X;
  g.lda = ldx;
  g.B = W;
  g.ldb = ldw;
  g.alpha = 1.f;
  g.beta = 0.f;
  g.ce_tgt = tgt;
  g.ce_v0 = v0;
  return g;
}

}  // namespace
}  // namespace nl

using namespace nl;

extern "C" size_t nl_lce_ws_bytes(int M, int V) {
  if (M <= 0 || V <= 0) return 0;
  return (size_t)M * lce_tiles_n(V) * 2 * sizeof(float) + (size_t)M * sizeof(float);
}

extern "C" int nl_lce_fwd(void* stream, int M, int D, int V, const nl_bf16* X, int64_t ldx, const nl_bf16* W,
                          int64_t ldw, const int32_t* targets, float* loss, float* lse, void* ws, size_t ws_bytes) {
  int rc = check_lce_args(M, D, V, X, ldx, W, ldw, targets);
  if (rc != NL_OK) return rc;
  if (M == 0) return NL_OK;
  if (!loss || !lse || !ws) return nl_set_error(NL_EINVAL, "lce_fwd: null pointer");
  if (((uintptr_t)ws & 15) != 0) return nl_set_error(NL_EALIGN, "lce_fwd: ws must be 16-byte aligned");
  if (ws_bytes < nl_lce_ws_bytes(M, V)) return nl_set_error(NL_EINVAL, "lce_fwd: workspace smaller than nl_lce_ws_bytes()");
  hipStream_t st = (hipStream_t)stream;
  GemmArgs g = lce_args(M, D, V, X, ldx, W, ldw, targets, 0);
  const int tn = lce_tiles_n(V);
  g.ce_part = static_cast<float*>(ws);
  g.ce_correct = g.ce_part + (size_t)M * tn * 2;
  launch_lce<kEpiCeStats>(g, st);
  hipLaunchKernelGGL(lce_merge_kernel, dim3((M + 3) / 4), dim3(256), 0, st, M, V, tn,
                     reinterpret_cast<const float2*>(g.ce_part), (const float*)g.ce_correct, targets, loss, lse);
  return nl_check_launch("nl_lce_fwd");
}

extern "C" int nl_lce_bwd_dlogits(void* stream, int M, int D, int V, int v0, int vn, const nl_bf16* X, int64_t ldx,
                                  const nl_bf16* W, int64_t ldw, const int32_t* targets, const float* lse,
                                  float scale, const float* scale_dev, nl_bf16* dlogits, int64_t ld_dlogits) {
  int rc = check_lce_args(M, D, V, X, ldx, W, ldw, targets);
  if (rc != NL_OK) return rc;
  if (v0 < 0 || vn < 0 || v0 > V - vn || (v0 & 7) != 0)
    return nl_set_error(NL_EINVAL, "lce_bwd: need 0 <= v0, v0 + vn <= V and v0 % 8 == 0");
  if (M == 0 || vn == 0) return NL_OK;
  if (!lse || !dlogits) return nl_set_error(NL_EINVAL, "lce_bwd: null pointer");
  if (ld_dlogits < vn || (ld_dlogits & 7) != 0 || ((uintptr_t)dlogits & 15) != 0)
    return nl_set_error(NL_EALIGN, "lce_bwd: dlogits 16-byte aligned with ld_dlogits >= vn, a multiple of 8");
  GemmArgs g = lce_args(M, D, vn, X, ldx, W + v0, ldw, targets, v0);
  g.C = dlogits;
  g.ldc = ld_dlogits;
  g.ce_lse = lse;
  g.ce_scale = scale;
  g.ce_scale_dev = scale_dev;
  launch_lce<kEpiCeGrad>(g, (hipStream_t)stream);
  return nl_check_launch("nl_lce_bwd_dlogits");
}

extern "C" size_t nl_gemm_ws_bytes(int opA, int opB, int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if ((opA != NL_OP_N && opA != NL_OP_T) || (opB != NL_OP_N && opB != NL_OP_T)) return 0;
  // the largest split workspace of the sub-products the call will run, for
  // dense operands (leading dimensions rounded up to 8)
  GemmArgs g{};
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = ((opA == NL_OP_N ? (int64_t)K : M) + 7) / 8 * 8;
  g.ldb = ((opB == NL_OP_N ? (int64_t)N : K) + 7) / 8 * 8;
  g.ldc = ((int64_t)N + 7) / 8 * 8;
  g.epi = NL_EPI_NONE;
  size_t most = make_plan(opA, opB, M, N, K, NL_EPI_NONE).ws_bytes;
  for_each_subproduct(opA, opB, g, NL_DTYPE_F32, [&](const GemmArgs& s) {
    most = std::max(most, make_plan(opA, opB, s.M, s.N, s.K, NL_EPI_NONE).ws_bytes);
    return NL_OK;
  });
  return most;
}

extern "C" int nl_gemm_fused(void* stream, int opA, int opB, int M, int N, int K, float alpha, const nl_bf16* A,
                             int64_t lda, const nl_bf16* B, int64_t ldb, float beta, void* C, int c_dtype, int64_t ldc,
                             const float* alpha_dev, int epi, const float* bias, nl_bf16* aux, int64_t ldaux, void* ws,
                             size_t ws_bytes) {
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
  if (epi < NL_EPI_NONE || epi > NL_EPI_DGELU) return nl_set_error(NL_EINVAL, "gemm: unknown epilogue");
  if ((epi == NL_EPI_BIAS || epi == NL_EPI_BIAS_GELU) && (!bias || ((uintptr_t)bias & 15) != 0))
    return nl_set_error(NL_EINVAL, "gemm: bias epilogue needs a 16-byte aligned fp32 bias[N]");
  if (epi == NL_EPI_BIAS_GELU || epi == NL_EPI_DGELU) {
    if (!aux || ((uintptr_t)aux & 15) != 0 || ldaux < N || (ldaux & 7) != 0)
      return nl_set_error(NL_EINVAL, "gemm: GELU epilogue needs a 16-byte aligned bf16 aux with ldaux >= N, ldaux % 8 == 0");
    if (beta != 0.f) return nl_set_error(NL_EINVAL, "gemm: GELU epilogues need beta == 0");
  }

  GemmArgs g{};
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
  g.epi = epi;
  g.bias = bias;
  g.aux = aux;
  g.ldaux = ldaux;
  hipStream_t st = (hipStream_t)stream;
  // validate the whole decomposition before launching any part of it
  int rc = for_each_subproduct(opA, opB, g, c_dtype, [](const GemmArgs&) { return NL_OK; });
  if (rc) return rc;
  rc = for_each_subproduct(opA, opB, g, c_dtype, [&](const GemmArgs& s) {
    Plan p = make_plan(opA, opB, s.M, s.N, s.K, s.epi);
    if (p.splits > 1 && (!ws || ws_bytes < p.ws_bytes || ((uintptr_t)ws & 15) != 0)) {
      // no (usable) workspace: one workgroup per tile over the whole K range
      p.splits = 1;
      p.k_chunk = s.K > 0 ? s.K : 1;
      p.ws_bytes = 0;
    }
    GemmArgs t = s;
    t.ws = static_cast<float*>(ws);
    if (c_dtype == NL_DTYPE_F32) launch_typed<float>(opA, opB, t, p, st);
    else launch_typed<uint16_t>(opA, opB, t, p, st);
    return NL_OK;
  });
  if (rc) return rc;
  return nl_check_launch("nl_gemm");
}

extern "C" int nl_gemm_ex(void* stream, int opA, int opB, int M, int N, int K, float alpha, const nl_bf16* A,
                          int64_t lda, const nl_bf16* B, int64_t ldb, float beta, void* C, int c_dtype, int64_t ldc,
                          const float* alpha_dev, void* ws, size_t ws_bytes) {
  return nl_gemm_fused(stream, opA, opB, M, N, K, alpha, A, lda, B, ldb, beta, C, c_dtype, ldc, alpha_dev,
                       NL_EPI_NONE, nullptr, nullptr, 0, ws, ws_bytes);
}

extern "C" int nl_gemm(void* stream, int opA, int opB, int M, int N, int K, float alpha, const nl_bf16* A,
                       int64_t lda, const nl_bf16* B, int64_t ldb, float beta, void* C, int c_dtype, int64_t ldc,
                       const float* alpha_dev) {
  return nl_gemm_ex(stream, opA, opB, M, N, K, alpha, A, lda, B, ldb, beta, C, c_dtype, ldc, alpha_dev, nullptr, 0);
}
