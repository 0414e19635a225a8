// flash.hip — causal FlashAttention for gfx950, head dim 64, bf16 in/out,
// fp32 softmax and accumulation, O(seq) memory in both directions.
//
// Algorithm (what the reference computes; nlearn/attention.py:82-131,
// iree_metal/kernels/flash_attention.metal:55-347):
//   forward   S = scale Q K^T (+ causal mask), online softmax, O = P V / l,
//             L = m + log l (natural log)
//   backward  D = rowsum(dO o O); P = exp(scale Q K^T - L);
//             dV = P^T dO; dP = dO V^T; dS = P o (dP - D);
//             dQ = scale dS K; dK = scale dS^T Q
//
// MI355X design
//   * v_mfma_f32_32x32x16_bf16 throughout; one workgroup = 4 waves = 128 rows
//     (queries in forward / dQ, keys in dK/dV), each wave owns 32 rows that
//     map to the 32 MFMA columns, so every lane owns exactly one row: the
//     online softmax (max, sum, rescale) is lane-local plus one swap with the
//     partner lane that holds the other 16 keys of the same row.
//   * Transposed products (S^T = K Q^T, O^T = V^T P^T, ...) keep that lane
//     ownership and let P / dS feed the next MFMA straight from registers: the
//     MFMA contraction order is permuted to match the accumulator layout
//     (lane group g holds keys {4g..4g+3, 8+4g..8+4g+3} of every 16), and the
//     operand read from LDS uses the same permutation.
//   * Tiles that must be read along the sequence (V for PV, K for dQ, Q and dO
//     for dK/dV) are stored transposed in LDS: 2x8 register transposes with
//     v_perm_b32 on the way in, 8-byte XOR swizzle (conflict-free fragment
//     reads). Row tiles use the same 16-byte XOR swizzle as the GEMM.
//   * 64-row K/V (or Q/dO) blocks are double buffered: the next block's global
//     loads are in flight while the current one is consumed.
//   * Causal work skipping per wave; fully masked waves only join the barriers.
//     The heaviest tiles are launched first.
#include <type_traits>
#include <atomic>
#include <mutex>

#include "common.h"

namespace nl {
namespace {

constexpr int kD = 64;        // head dim
constexpr int kRows = 128;    // rows per workgroup (4 waves x 32)
constexpr int kBlk = 64;      // rows per streamed block
constexpr int kThreads = 256;

__device__ __forceinline__ int swz16(int row, int kc) { return kc ^ ((row ^ (row >> 3)) & 7); }

// ---- 64x64 bf16 tile, row layout: element (r, c) at r*64 + swz16(r, c/8)*8 + c%8
struct RowTile {
  u32x4 r[2];
  __device__ __forceinline__ void load(const uint16_t* base, int64_t rstride, int rows_valid, int tid) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int u = i * kThreads + tid;
      const int row = u >> 3, kc = u & 7;
      if (row < rows_valid) r[i] = *reinterpret_cast<const u32x4*>(base + (int64_t)row * rstride + kc * 8);
      else r[i] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  __device__ __forceinline__ void store(uint16_t* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int u = i * kThreads + tid;
      const int row = u >> 3, kc = u & 7;
      *reinterpret_cast<u32x4*>(lds + row * 64 + swz16(row, kc) * 8) = r[i];
    }
  }
};
__device__ __forceinline__ bf16x8 row_frag(const uint16_t* lds, int row, int kc) {
  return as_bf16x8(*reinterpret_cast<const u32x4*>(lds + row * 64 + swz16(row, kc) * 8));
}

// ---- 64x64 tile stored transposed: global (r, c) -> LDS (c, r);
// element (c, r) at c*64 + ((r/4) ^ (c & 15))*4 + r%4
struct TransTile {
  u32x4 r[2];  // rows 2p, 2p+1 of an 8-column block
  __device__ __forceinline__ void load(const uint16_t* base, int64_t rstride, int rows_valid, int tid) {
    const int rp = tid >> 3, cb = tid & 7;  // row pair 0..31, column block 0..7
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = rp * 2 + i;
      if (row < rows_valid) r[i] = *reinterpret_cast<const u32x4*>(base + (int64_t)row * rstride + cb * 8);
      else r[i] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  __device__ __forceinline__ void store(uint16_t* lds, int tid) const {
    const int rp = tid >> 3, cb = tid & 7;
    const int r0 = rp * 2;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
      const uint32_t w = __builtin_amdgcn_perm(r[1][c >> 1], r[0][c >> 1], sel);  // (row r0, row r0+1) at col
      const int col = cb * 8 + c;
      *reinterpret_cast<uint32_t*>(lds + col * 64 + (((r0 >> 2) ^ (col & 15)) << 2) + (r0 & 3)) = w;
    }
  }
};
// Operand of a 32x32x16 MFMA read from a transposed tile: row `c` (lane%32),
// sequence positions {base+4g..+3, base+8+4g..+3} (the permuted k order).
__device__ __forceinline__ bf16x8 trans_frag(const uint16_t* lds, int c, int base, int g) {
  const int h0 = (base >> 2) + g, h1 = h0 + 2;
  const u32x2 lo = *reinterpret_cast<const u32x2*>(lds + c * 64 + ((h0 ^ (c & 15)) << 2));
  const u32x2 hi = *reinterpret_cast<const u32x2*>(lds + c * 64 + ((h1 ^ (c & 15)) << 2));
  return as_bf16x8(u32x4{lo[0], lo[1], hi[0], hi[1]});
}
// 8 accumulator values (registers 8h..8h+7 of a 32x32 tile) as a bf16 operand.
__device__ __forceinline__ bf16x8 pack_frag(const f32x16& a, int h) {
  u32x4 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = pack_bf16x2(a[8 * h + 2 * j], a[8 * h + 2 * j + 1]);
  return as_bf16x8(v);
}
// 8 bf16 of one row straight from global memory (16 bytes), zero if !valid.
__device__ __forceinline__ bf16x8 global_frag(const uint16_t* p, bool valid) {
  if (!valid) return as_bf16x8(u32x4{0u, 0u, 0u, 0u});
  return as_bf16x8(*reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void zero(f32x16& a) {
#pragma unroll
  for (int r = 0; r < 16; ++r) a[r] = 0.f;
}

// ---- DMA path: 64 x 64 bf16 tiles filled straight from global memory into LDS
// (buffer_load ... lds): 128-byte rows of eight 16-byte chunks, chunk c of row k
// at slot c ^ swz(k). The one swizzle serves both ways a tile is read:
//   * 16-byte reads of one chunk down 16 consecutive rows (MFMA fragments along
//     a row): the 8 even rows get 8 distinct slots, the odd rows sit in the
//     other half of the banks;
//   * ds_read_b64_tr_b16 over 4 consecutive rows x 4 chunks per 32 lanes
//     (MFMA fragments down a column): rows k and k+2 map the 4-chunk group to
//     disjoint slots.
__device__ __forceinline__ int swz(int k) { return (((k >> 1) & 1) << 2) | ((k >> 2) & 3); }
// Tiles read one way only (the forward's K along rows, V down columns) use the
// cheaper single-purpose swizzles (fewer distinct fragment addresses to keep).
__device__ __forceinline__ int swz_rows(int k) { return (k ^ (k >> 3)) & 7; }
__device__ __forceinline__ int swz_cols(int k) { return ((k >> 1) & 1) << 2; }
enum Swz { kBoth, kAlongRows, kDownCols };
template <int W>
__device__ __forceinline__ int swz_of(int k) {
  if constexpr (W == kAlongRows) return swz_rows(k);
  else if constexpr (W == kDownCols) return swz_cols(k);
  else return swz(k);
}

// DMA rows row0 .. row0+63 (row stride ld elements) of the buffer into a tile:
// 4 waves x 2 instructions x 64 lanes x 16 bytes. Rows past the buffer's end
// read as zero.
template <int W = kBoth>
__device__ __forceinline__ void dma_tile(__amdgpu_buffer_rsrc_t rs, uint16_t* lds, int row0, int64_t ld, int wave,
                                         int lane) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int blk = i * 4 + wave;           // 1 KB of the tile = 8 rows
    const int u = blk * 64 + lane;          // destination chunk
    const int r = u >> 3, slot = u & 7;
    const int c = slot ^ swz_of<W>(r);
    dma16(rs, lds + blk * 512, (uint32_t)(((int64_t)(row0 + r) * ld + c * 8) * 2), 0);
  }
}
// 8 consecutive columns c*8.. of row r
template <int W = kBoth>
__device__ __forceinline__ bf16x8 frag_R(const uint16_t* t, int r, int c) {
  return as_bf16x8(*reinterpret_cast<const u32x4*>(t + r * 64 + ((c ^ swz_of<W>(r)) << 3)));
}
// MFMA operand down the columns of a tile [k][mn]: lane (mn = mnb + lane%32, g = lane/32) gets
// t[k][mn] for k = kb + {4g..4g+3, 8+4g..8+4g+3} -- the permuted k order that
// matches pack_frag of a 32x32 accumulator.
template <int W = kBoth>
__device__ __forceinline__ bf16x8 frag_T(const uint16_t* t, int mnb, int kb, int lane) {
  const int G = lane >> 4, j = lane & 15;
  const int mn = mnb + 16 * (G & 1) + 4 * (j & 3);
  const int k0 = kb + 4 * (G >> 1) + (j >> 2);
  const int k1 = k0 + 8;
  const u32x2 lo = ds_read_tr16(t + k0 * 64 + (((mn >> 3) ^ swz_of<W>(k0)) << 3) + (mn & 7));
  const u32x2 hi = ds_read_tr16(t + k1 * 64 + (((mn >> 3) ^ swz_of<W>(k1)) << 3) + (mn & 7));
  return as_bf16x8(u32x4{lo[0], lo[1], hi[0], hi[1]});
}
// Buffer resource over rows 0 .. S-1 of one head (row stride ld, 64 columns).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_rsrc(const uint16_t* p, int S, int64_t ld) {
  return make_rsrc(p, (uint32_t)((((int64_t)(S - 1)) * ld + 64) * 2));
}

struct Op {
  const uint16_t* p;
  nl_attn_stride s;
  __device__ __forceinline__ const uint16_t* at(int b, int h, int row) const {
    return p + (int64_t)b * s.batch + (int64_t)h * s.head + (int64_t)row * s.row;
  }
};
struct OutOp {
  uint16_t* p;
  nl_attn_stride s;
  __device__ __forceinline__ uint16_t* at(int b, int h, int row) const {
    return p + (int64_t)b * s.batch + (int64_t)h * s.head + (int64_t)row * s.row;
  }
};

// Workgroup id -> (tile rank, head, batch) over a 1-D grid with the rank
// slowest. The hardware deals consecutive workgroups to the 8 XCDs in turn, so
// every rank (causal work per tile grows with it, up to ntiles x) spreads
// evenly over the XCDs and their CUs. With the tile index fastest and a
// power-of-two tile count, all the heaviest tiles would land on the same XCDs.
struct TileCoord {
  int rank, h, b;
};
__device__ __forceinline__ TileCoord tile_coord(int H, int B) {
  const int bh = H * B;
  const int id = (int)blockIdx.x;
  TileCoord t;
  t.rank = id / bh;
  const int r = id - t.rank * bh;
  t.b = r / H;
  t.h = r - t.b * H;
  return t;
}

struct FwdArgs {
  int S, causal, H, B;
  float scale_log2;
  Op q, k, v;
  OutOp o;
  float* L;
};

// Store a wave's 32 rows x 64 columns (a transposed accumulator pair: lane
// (row l32, g) holds columns dt*32 + 8qq + 4g + t in acc[dt][4qq + t]) through
// a 4 KB LDS slab, so that each store instruction writes
// whole 128-byte rows (16 bytes per lane) instead of 8 bytes in each of 32 rows.
// Slab row r holds its 16-byte chunk c at slot c ^ (r & 7). Rows at or past S
// are not stored. The caller makes sure no other wave still reads the slab.
__device__ __forceinline__ void store_rows_staged(uint16_t* slab, const f32x16 acc[2], float mul, int g, int l32,
                                                  int lane, const OutOp& out, int b, int h, int row0, int S) {
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int c = dt * 4 + qq;  // columns 8c + 4g .. 8c + 4g + 3
      *reinterpret_cast<u32x2*>(slab + l32 * 64 + ((c ^ (l32 & 7)) << 3) + 4 * g) =
          u32x2{pack_bf16x2(acc[dt][4 * qq] * mul, acc[dt][4 * qq + 1] * mul),
                pack_bf16x2(acc[dt][4 * qq + 2] * mul, acc[dt][4 * qq + 3] * mul)};
    }
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int r = it * 8 + (lane >> 3), c = lane & 7;
    const u32x4 v = *reinterpret_cast<const u32x4*>(slab + r * 64 + ((c ^ (r & 7)) << 3));
    if (row0 + r < S) *reinterpret_cast<u32x4*>(out.at(b, h, row0 + r) + c * 8) = v;
  }
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads, 4) void flash_fwd_kernel(FwdArgs a) {
  // double-buffered K and V blocks; every buffer its own
  // LDS object so the DMA of block kb+1 never makes the reads of block kb wait
  __shared__ __attribute__((aligned(16))) uint16_t sK0[kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sK1[kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sV0[kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sV1[kBlk * kD];
  const int S = a.S;
  const int nqt = (S + kRows - 1) / kRows;
  const TileCoord tc = tile_coord(a.H, a.B);
  const int qt = nqt - 1 - tc.rank;  // heaviest (latest) query tiles first
  const int h = tc.h, b = tc.b;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int qw0 = qt * kRows + wave * 32;  // first query of this wave
  const int q = qw0 + l32;                 // this lane's query
  const bool qvalid = q < S;

  bf16x8 qf[4];
  {
    const uint16_t* qp = a.q.at(b, h, qvalid ? q : 0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[ks] = global_frag(qp + ks * 16 + g * 8, qvalid);
  }

  const int kend_wg = a.causal ? min(S, qt * kRows + kRows) : S;
  const int kend_w = a.causal ? min(S, qw0 + 32) : S;
  const int nkb = (kend_wg + kBlk - 1) / kBlk;
  const __amdgpu_buffer_rsrc_t rk = head_rsrc(a.k.at(b, h, 0), S, a.k.s.row);
  const __amdgpu_buffer_rsrc_t rv = head_rsrc(a.v.at(b, h, 0), S, a.v.s.row);
  auto issue = [&](uint16_t* sk, uint16_t* sv, int kb) {
    dma_tile<kAlongRows>(rk, sk, kb * kBlk, a.k.s.row, wave, lane);
    dma_tile<kDownCols>(rv, sv, kb * kBlk, a.v.s.row, wave, lane);
  };

  const float c = a.scale_log2;  // scores are kept raw; exp2 arguments are c * s - m
  constexpr float kSlack = 8.f;
  float m = -INFINITY, l = 0.f;  // exponent base (scaled, log2 units) and this lane's partial sum
  f32x16 o[2];
  zero(o[0]);
  zero(o[1]);

  auto compute = [&](const uint16_t* sk, const uint16_t* sv, int kb) {
    const int k0 = kb * kBlk;
    if (k0 >= kend_w) return;  // every query of this wave precedes the block
    // S^T (keys x queries): lane (query, g) holds keys k0 + kt*32 + 8(r/4) + 4g + r%4
    f32x16 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      zero(s[kt]);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) s[kt] = mfma32(frag_R<kAlongRows>(sk, kt * 32 + l32, ks * 2 + g), qf[ks], s[kt]);
    }
    // One uniform branch per block between a masked and an unmasked variant
    // (a per-element test of a uniform flag compiles to one branch per score).
    const bool need_mask = (a.causal && k0 + kBlk - 1 > qw0) || (k0 + kBlk > S);
    float bm = -INFINITY;
    auto mask_max = [&](auto masked) {
      const int lim = a.causal ? min(q, S - 1) : S - 1;  // last visible key
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = s[kt][r];
          if constexpr (decltype(masked)::value) {
            if (k0 + kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3) > lim) x = -INFINITY;
          }
          s[kt][r] = x;
          bm = fmaxf(bm, x);
        }
    };
    if (need_mask) mask_max(std::true_type{});
    else mask_max(std::false_type{});
    bm = fmaxf(bm, __shfl_xor(bm, 32, kWave));
    // The exponent base m moves only when the block max exceeds it by more
    // than kSlack (log2 units). Probabilities then stay below 2^kSlack (bf16
    // and fp32 hold them without loss of relative precision), and once the
    // base has settled most blocks skip the rescale of O and l below.
    const float cand = bm * c;
    const bool up = cand > m + kSlack;
    const float mn = up ? cand : m;
    const float alpha = up ? ((m == -INFINITY) ? 0.f : fast_exp2(m - mn)) : 1.f;
    const float nmn = (mn == -INFINITY) ? 0.f : -mn;
    float rs = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(__builtin_fmaf(s[kt][r], c, nmn));  // -inf -> 0
        s[kt][r] = p;
        rs += p;
      }
    l = __builtin_fmaf(l, alpha, rs);
    m = mn;
    // alpha == 1 exactly when the base did not move: whole blocks then skip
    // the rescale
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
    }
    // O^T (d x queries) += V^T P^T, P straight from the registers
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const bf16x8 pf = pack_frag(s[kt], hh);
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
          o[dt] = mfma32(frag_T<kDownCols>(sv, dt * 32, kt * 32 + hh * 16, lane), pf, o[dt]);
      }
  };

  if (nkb > 0) issue(sK0, sV0, 0);
  for (int kb = 0; kb < nkb; kb += 2) {
    wait_vm<0>();
    __syncthreads();
    if (kb + 1 < nkb) issue(sK1, sV1, kb + 1);
    compute(sK0, sV0, kb);
    if (kb + 1 >= nkb) break;
    wait_vm<0>();
    __syncthreads();
    if (kb + 2 < nkb) issue(sK0, sV0, kb + 2);
    compute(sK1, sV1, kb + 1);
  }

  const float lt = l + __shfl_xor(l, 32, kWave);
  const float inv = qvalid ? 1.f / lt : 0.f;
  if (qvalid && g == 0) a.L[((int64_t)b * a.H + h) * S + q] = (m + fast_log2(lt)) * kLn2;
  __syncthreads();  // every wave is done reading the K / V blocks
  store_rows_staged(wave == 0 ? sK0 : wave == 1 ? sK1 : wave == 2 ? sV0 : sV1, o, inv, g, l32, lane, a.o, b, h, qw0,
                    S);
}

// ---------------------------------------------------------------------------
// backward preprocess: D = rowsum(dO o O)
// ---------------------------------------------------------------------------
struct PreArgs {
  int S, H;
  Op o, dout;
  float* D;
};
// grid (ceil(S / 32), H, B): 32 rows per workgroup, 8 lanes per row, 16 bytes
// of O and of dO per lane; no division in the index math
__global__ __launch_bounds__(256) void flash_bwd_pre_kernel(PreArgs a) {
  const int s = (int)blockIdx.x * 32 + ((int)threadIdx.x >> 3);
  const int part = (int)threadIdx.x & 7;
  const int h = (int)blockIdx.y, b = (int)blockIdx.z;
  float acc = 0.f;
  if (s < a.S) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(a.o.at(b, h, s) + part * 8);
    const u32x4 y = *reinterpret_cast<const u32x4*>(a.dout.at(b, h, s) + part * 8);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += bf16_lo(x[j]) * bf16_lo(y[j]) + bf16_hi(x[j]) * bf16_hi(y[j]);
  }
  acc += __shfl_xor(acc, 1, kWave);
  acc += __shfl_xor(acc, 2, kWave);
  acc += __shfl_xor(acc, 4, kWave);
  if (s < a.S && part == 0) a.D[((int64_t)b * a.H + h) * a.S + s] = acc;
}

struct BwdArgs {
  int S, causal, H, B;
  float scale, scale_log2;
  Op q, k, v, dout;
  const float* L;  // natural-log lse
  const float* D;
  OutOp dq, dk, dv;
};

// ---------------------------------------------------------------------------
// dK, dV: workgroup = 128 keys, streams 64-query blocks from the diagonal on.
// Per block the Q and dO tiles (and L, D) arrive by DMA; each tile is read both
// along rows (S = Q K^T, dP = dO V^T) and down columns (dV += dO^T P,
// dK += Q^T dS) from the one LDS copy.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads, 2) void flash_bwd_dkdv_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sQ0[kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sQ1[kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sO0[kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sO1[kBlk * kD];
  __shared__ __attribute__((aligned(16))) float sL0[kBlk];
  __shared__ __attribute__((aligned(16))) float sL1[kBlk];
  __shared__ __attribute__((aligned(16))) float sD0[kBlk];
  __shared__ __attribute__((aligned(16))) float sD1[kBlk];
  const int S = a.S;
  const TileCoord tc = tile_coord(a.H, a.B);
  const int kt_idx = tc.rank;  // low key tiles see the most queries: launched first
  const int h = tc.h, b = tc.b;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int kw0 = kt_idx * kRows + wave * 32;
  const int key = kw0 + l32;
  const bool kvalid = key < S;
  const int64_t lbase = ((int64_t)b * a.H + h) * S;

  bf16x8 kf[4], vf[4];
  {
    const uint16_t* kp = a.k.at(b, h, kvalid ? key : 0);
    const uint16_t* vp = a.v.at(b, h, kvalid ? key : 0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      kf[ks] = global_frag(kp + ks * 16 + g * 8, kvalid);
      vf[ks] = global_frag(vp + ks * 16 + g * 8, kvalid);
    }
  }
  f32x16 dk[2], dv[2];
  zero(dk[0]);
  zero(dk[1]);
  zero(dv[0]);
  zero(dv[1]);

  const int qstart = a.causal ? (kt_idx * kRows) / kBlk * kBlk : 0;
  const int nqb = (S - qstart + kBlk - 1) / kBlk;
  const __amdgpu_buffer_rsrc_t rq = head_rsrc(a.q.at(b, h, 0), S, a.q.s.row);
  const __amdgpu_buffer_rsrc_t ro = head_rsrc(a.dout.at(b, h, 0), S, a.dout.s.row);
  const __amdgpu_buffer_rsrc_t rl = make_rsrc(a.L + lbase, (uint32_t)S * 4u);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.D + lbase, (uint32_t)S * 4u);
  auto issue = [&](uint16_t* sq, uint16_t* so, float* sl, float* sd, int qb) {
    const int q0 = qstart + qb * kBlk;
    dma_tile(rq, sq, q0, a.q.s.row, wave, lane);
    dma_tile(ro, so, q0, a.dout.s.row, wave, lane);
    if (lane < 16) {  // 64 floats of L (wave 0) and of D (wave 1); rows past S read zero
      if (wave == 0) dma16(rl, sl, (uint32_t)(q0 + lane * 4) * 4u, 0);
      if (wave == 1) dma16(rd, sd, (uint32_t)(q0 + lane * 4) * 4u, 0);
    }
  };
  const float c = a.scale_log2;

  auto compute = [&](const uint16_t* sq, const uint16_t* so, const float* sl, const float* sd, int qb) {
    const int q0 = qstart + qb * kBlk;
    // this wave's keys see queries >= kw0 only (causal)
    if (a.causal && q0 + kBlk - 1 < kw0) return;
    const bool need_mask = (a.causal && q0 < kw0 + 31) || (q0 + kBlk > S);
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      // dP - D straight from the product: its accumulator starts at -D
      f32x16 s, dp;
      zero(s);
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const f32x4 nD4 = *reinterpret_cast<const f32x4*>(sd + qt * 32 + qq * 8 + 4 * g);
#pragma unroll
        for (int t = 0; t < 4; ++t) dp[4 * qq + t] = nD4[t];
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        s = mfma32(frag_R(sq, qt * 32 + l32, ks * 2 + g), kf[ks], s);
        dp = mfma32(frag_R(so, qt * 32 + l32, ks * 2 + g), vf[ks], dp);
      }
      // lane (key, g) holds query rows qt*32 + 8qq + 4g + t
      auto probs = [&](auto masked) {
        const int lo = a.causal ? key : 0;  // first query that sees this key
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int qr = qt * 32 + qq * 8 + 4 * g;
          const f32x4 nL4 = *reinterpret_cast<const f32x4*>(sl + qr);  // -L log2(e)
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int r = 4 * qq + t;
            float p = fast_exp2(__builtin_fmaf(s[r], c, nL4[t]));
            if constexpr (decltype(masked)::value) {
              const int qi = q0 + qr + t;
              if (qi >= S || qi < lo) p = 0.f;
            }
            s[r] = p;
            dp[r] = p * dp[r];
          }
        }
      };
      if (need_mask) probs(std::true_type{});
      else probs(std::false_type{});
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const bf16x8 pf = pack_frag(s, hh);
        const bf16x8 dsf = pack_frag(dp, hh);
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          dv[dt] = mfma32(frag_T(so, dt * 32, qt * 32 + hh * 16, lane), pf, dv[dt]);
          dk[dt] = mfma32(frag_T(sq, dt * 32, qt * 32 + hh * 16, lane), dsf, dk[dt]);
        }
      }
    }
  };

  // Once a block's L and D have landed, the lanes that fetched them rewrite
  // them in place as -L log2(e) and -D (one vector op each per block instead of
  // one per score in every wave).
  auto prep = [&](float* sl, float* sd) {
    if (lane < 16 && wave < 2) {
      float* p = (wave == 0 ? sl : sd) + lane * 4;
      const float f = wave == 0 ? -kLog2e : -1.f;
      f32x4 x = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] *= f;
      *reinterpret_cast<f32x4*>(p) = x;
    }
  };
  if (nqb > 0) issue(sQ0, sO0, sL0, sD0, 0);
  for (int qb = 0; qb < nqb; qb += 2) {
    wait_vm<0>();
    prep(sL0, sD0);
    __syncthreads();
    if (qb + 1 < nqb) issue(sQ1, sO1, sL1, sD1, qb + 1);
    compute(sQ0, sO0, sL0, sD0, qb);
    if (qb + 1 >= nqb) break;
    wait_vm<0>();
    prep(sL1, sD1);
    __syncthreads();
    if (qb + 2 < nqb) issue(sQ0, sO0, sL0, sD0, qb + 2);
    compute(sQ1, sO1, sL1, sD1, qb + 1);
  }
  __syncthreads();  // every wave is done reading the Q / dO blocks
  uint16_t* slab = wave == 0 ? sQ0 : wave == 1 ? sQ1 : wave == 2 ? sO0 : sO1;
  store_rows_staged(slab, dk, a.scale, g, l32, lane, a.dk, b, h, kw0, S);
  store_rows_staged(slab + 32 * kD, dv, 1.f, g, l32, lane, a.dv, b, h, kw0, S);
}

// ---------------------------------------------------------------------------
// dQ: workgroup = 128 queries, streams 64-key blocks up to the diagonal; the
// K tile is read along rows (S) and down columns (dQ += dS K).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads, 3) void flash_bwd_dq_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sK0[kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sK1[kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sV0[kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sV1[kBlk * kD];
  const int S = a.S;
  const int nqt = (S + kRows - 1) / kRows;
  const TileCoord tc = tile_coord(a.H, a.B);
  const int qt = nqt - 1 - tc.rank;
  const int h = tc.h, b = tc.b;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int qw0 = qt * kRows + wave * 32;
  const int q = qw0 + l32;
  const bool qvalid = q < S;
  const int64_t lbase = ((int64_t)b * a.H + h) * S;

  bf16x8 qf[4], df[4];
  {
    const uint16_t* qp = a.q.at(b, h, qvalid ? q : 0);
    const uint16_t* dp = a.dout.at(b, h, qvalid ? q : 0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qf[ks] = global_frag(qp + ks * 16 + g * 8, qvalid);
      df[ks] = global_frag(dp + ks * 16 + g * 8, qvalid);
    }
  }
  const float c = a.scale_log2;
  const float nLq = qvalid ? -a.L[lbase + q] * kLog2e : -INFINITY;
  const float Dq = qvalid ? a.D[lbase + q] : 0.f;

  const int kend_wg = a.causal ? min(S, qt * kRows + kRows) : S;
  const int kend_w = a.causal ? min(S, qw0 + 32) : S;
  const int nkb = (kend_wg + kBlk - 1) / kBlk;
  const __amdgpu_buffer_rsrc_t rk = head_rsrc(a.k.at(b, h, 0), S, a.k.s.row);
  const __amdgpu_buffer_rsrc_t rv = head_rsrc(a.v.at(b, h, 0), S, a.v.s.row);
  auto issue = [&](uint16_t* sk, uint16_t* sv, int kb) {
    dma_tile(rk, sk, kb * kBlk, a.k.s.row, wave, lane);
    dma_tile(rv, sv, kb * kBlk, a.v.s.row, wave, lane);
  };

  f32x16 dq[2];
  zero(dq[0]);
  zero(dq[1]);

  auto compute = [&](const uint16_t* sk, const uint16_t* sv, int kb) {
    const int k0 = kb * kBlk;
    if (k0 >= kend_w) return;
    const bool need_mask = (a.causal && k0 + kBlk - 1 > qw0) || (k0 + kBlk > S);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      f32x16 s, dp;
      zero(s);
      zero(dp);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        s = mfma32(frag_R(sk, kt * 32 + l32, ks * 2 + g), qf[ks], s);
        dp = mfma32(frag_R(sv, kt * 32 + l32, ks * 2 + g), df[ks], dp);
      }
      auto probs = [&](auto masked) {
        const int lim = a.causal ? min(q, S - 1) : S - 1;  // last visible key
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float p = fast_exp2(__builtin_fmaf(s[r], c, nLq));
          if constexpr (decltype(masked)::value) {
            if (k0 + kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3) > lim) p = 0.f;
          }
          dp[r] = p * (dp[r] - Dq);
        }
      };
      if (need_mask) probs(std::true_type{});
      else probs(std::false_type{});
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const bf16x8 dsf = pack_frag(dp, hh);
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) dq[dt] = mfma32(frag_T(sk, dt * 32, kt * 32 + hh * 16, lane), dsf, dq[dt]);
      }
    }
  };

  if (nkb > 0) issue(sK0, sV0, 0);
  for (int kb = 0; kb < nkb; kb += 2) {
    wait_vm<0>();
    __syncthreads();
    if (kb + 1 < nkb) issue(sK1, sV1, kb + 1);
    compute(sK0, sV0, kb);
    if (kb + 1 >= nkb) break;
    wait_vm<0>();
    __syncthreads();
    if (kb + 2 < nkb) issue(sK0, sV0, kb + 2);
    compute(sK1, sV1, kb + 1);
  }
  // Direct 8-byte stores (lane = row): measured faster here than staging
  // through LDS, which needs a barrier that makes the waves with less causal
  // work wait for the others.
  if (qvalid) {
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int col = dt * 32 + qq * 8 + 4 * g;
        *reinterpret_cast<u32x2*>(a.dq.at(b, h, q) + col) =
            u32x2{pack_bf16x2(dq[dt][4 * qq] * a.scale, dq[dt][4 * qq + 1] * a.scale),
                  pack_bf16x2(dq[dt][4 * qq + 2] * a.scale, dq[dt][4 * qq + 3] * a.scale)};
      }
  }
}

// ---------------------------------------------------------------------------
// host-side validation
// ---------------------------------------------------------------------------
bool stride_ok(const nl_attn_stride& s) { return ((s.batch | s.head | s.row) & 7) == 0 && s.row >= 64; }
// the DMA path addresses one head's rows with 32-bit byte offsets
bool extent_ok(int S, const nl_attn_stride& s) { return ((int64_t)S * s.row + 64) * 2 < ((int64_t)1 << 31); }

int check_common(int B, int H, int S, int d, int causal) {
  if (B < 0 || H < 0 || S < 0) return nl_set_error(NL_EINVAL, "flash: negative dimension");
  if (d != kD) return nl_set_error(NL_EUNSUPPORTED, "flash: d_head must be 64");
  if (causal != 0 && causal != 1) return nl_set_error(NL_EINVAL, "flash: causal must be 0 or 1");
  if (H > 65535 || B > 65535) return nl_set_error(NL_EINVAL, "flash: batch and heads must be <= 65535");
  return NL_OK;
}
int check_op(const void* p, const nl_attn_stride& s, const char* name) {
  if (!p) return nl_set_error(NL_EINVAL, std::string("flash: null ") + name);
  if (((uintptr_t)p & 15) != 0) return nl_set_error(NL_EALIGN, std::string("flash: ") + name + " not 16-byte aligned");
  if (!stride_ok(s))
    return nl_set_error(NL_EALIGN, std::string("flash: ") + name + " strides must be multiples of 8 (row >= 64)");
  return NL_OK;
}

}  // namespace
}  // namespace nl

using namespace nl;

#define NL_TRY(x)        \
  do {                   \
    int rc_ = (x);       \
    if (rc_) return rc_; \
  } while (0)

extern "C" int nl_flash_attention_fwd(void* stream, int batch, int heads, int seq, int d_head, float scale,
                                      int causal, const nl_bf16* Q, nl_attn_stride sq, const nl_bf16* K,
                                      nl_attn_stride sk, const nl_bf16* V, nl_attn_stride sv, nl_bf16* O,
                                      nl_attn_stride so, float* L) {
  NL_TRY(check_common(batch, heads, seq, d_head, causal));
  if (batch == 0 || heads == 0 || seq == 0) return NL_OK;
  NL_TRY(check_op(Q, sq, "Q"));
  NL_TRY(check_op(K, sk, "K"));
  NL_TRY(check_op(V, sv, "V"));
  NL_TRY(check_op(O, so, "O"));
  if (!L) return nl_set_error(NL_EINVAL, "flash: null L");
  if (!extent_ok(seq, sk) || !extent_ok(seq, sv))
    return nl_set_error(NL_EUNSUPPORTED, "flash: one head's K or V spans 2 GB or more");
  FwdArgs a;
  a.S = seq;
  a.causal = causal;
  a.scale_log2 = scale * kLog2e;
  a.q = Op{Q, sq};
  a.k = Op{K, sk};
  a.v = Op{V, sv};
  a.o = OutOp{O, so};
  a.L = L;
  a.H = heads;
  a.B = batch;
  const int64_t wgs = (int64_t)((seq + kRows - 1) / kRows) * heads * batch;
  if (wgs >= ((int64_t)1 << 31)) return nl_set_error(NL_EUNSUPPORTED, "flash: too many tiles");
  hipLaunchKernelGGL(flash_fwd_kernel, dim3((unsigned)wgs), dim3(kThreads), 0, (hipStream_t)stream, a);
  return nl_check_launch("nl_flash_attention_fwd");
}

extern "C" int nl_flash_attention_bwd_preprocess(void* stream, int batch, int heads, int seq, int d_head,
                                                 const nl_bf16* O, nl_attn_stride so, const nl_bf16* dO,
                                                 nl_attn_stride sdo, float* D) {
  NL_TRY(check_common(batch, heads, seq, d_head, 1));
  if (batch == 0 || heads == 0 || seq == 0) return NL_OK;
  NL_TRY(check_op(O, so, "O"));
  NL_TRY(check_op(dO, sdo, "dO"));
  if (!D) return nl_set_error(NL_EINVAL, "flash: null D");
  PreArgs a;
  a.S = seq;
  a.H = heads;
  a.o = Op{O, so};
  a.dout = Op{dO, sdo};
  a.D = D;
  hipLaunchKernelGGL(flash_bwd_pre_kernel, dim3((unsigned)((seq + 31) / 32), (unsigned)heads, (unsigned)batch),
                     dim3(256), 0, (hipStream_t)stream, a);
  return nl_check_launch("nl_flash_attention_bwd_preprocess");
}

static int fill_bwd(BwdArgs& a, int seq, int causal, float scale, const nl_bf16* Q, nl_attn_stride sq,
                    const nl_bf16* K, nl_attn_stride sk, const nl_bf16* V, nl_attn_stride sv, const nl_bf16* dO,
                    nl_attn_stride sdo, const float* L, const float* D) {
  NL_TRY(check_op(Q, sq, "Q"));
  NL_TRY(check_op(K, sk, "K"));
  NL_TRY(check_op(V, sv, "V"));
  NL_TRY(check_op(dO, sdo, "dO"));
  if (!L || !D) return nl_set_error(NL_EINVAL, "flash: null L or D");
  if (!extent_ok(seq, sq) || !extent_ok(seq, sk) || !extent_ok(seq, sv) || !extent_ok(seq, sdo))
    return nl_set_error(NL_EUNSUPPORTED, "flash: one head's Q, K, V or dO spans 2 GB or more");
  a.S = seq;
  a.causal = causal;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.q = Op{Q, sq};
  a.k = Op{K, sk};
  a.v = Op{V, sv};
  a.dout = Op{dO, sdo};
  a.L = L;
  a.D = D;
  return NL_OK;
}

static int bwd_grid(int batch, int heads, int seq, BwdArgs& a, dim3& grid) {
  a.H = heads;
  a.B = batch;
  const int64_t wgs = (int64_t)((seq + kRows - 1) / kRows) * heads * batch;
  if (wgs >= ((int64_t)1 << 31)) return nl_set_error(NL_EUNSUPPORTED, "flash: too many tiles");
  grid = dim3((unsigned)wgs);
  return NL_OK;
}

extern "C" int nl_flash_attention_bwd_dq(void* stream, int batch, int heads, int seq, int d_head, float scale,
                                         int causal, const nl_bf16* Q, nl_attn_stride sq, const nl_bf16* K,
                                         nl_attn_stride sk, const nl_bf16* V, nl_attn_stride sv,
                                         const nl_bf16* dO, nl_attn_stride sdo, const float* L, const float* D,
                                         nl_bf16* dQ, nl_attn_stride sdq) {
  NL_TRY(check_common(batch, heads, seq, d_head, causal));
  if (batch == 0 || heads == 0 || seq == 0) return NL_OK;
  BwdArgs a;
  NL_TRY(fill_bwd(a, seq, causal, scale, Q, sq, K, sk, V, sv, dO, sdo, L, D));
  NL_TRY(check_op(dQ, sdq, "dQ"));
  a.dq = OutOp{dQ, sdq};
  dim3 grid;
  NL_TRY(bwd_grid(batch, heads, seq, a, grid));
  hipLaunchKernelGGL(flash_bwd_dq_kernel, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
  return nl_check_launch("nl_flash_attention_bwd_dq");
}

extern "C" int nl_flash_attention_bwd_dkdv(void* stream, int batch, int heads, int seq, int d_head, float scale,
                                           int causal, const nl_bf16* Q, nl_attn_stride sq, const nl_bf16* K,
                                           nl_attn_stride sk, const nl_bf16* V, nl_attn_stride sv,
                                           const nl_bf16* dO, nl_attn_stride sdo, const float* L, const float* D,
                                           nl_bf16* dK, nl_attn_stride sdk, nl_bf16* dV, nl_attn_stride sdv) {
  NL_TRY(check_common(batch, heads, seq, d_head, causal));
  if (batch == 0 || heads == 0 || seq == 0) return NL_OK;
  BwdArgs a;
  NL_TRY(fill_bwd(a, seq, causal, scale, Q, sq, K, sk, V, sv, dO, sdo, L, D));
  NL_TRY(check_op(dK, sdk, "dK"));
  NL_TRY(check_op(dV, sdv, "dV"));
  a.dk = OutOp{dK, sdk};
  a.dv = OutOp{dV, sdv};
  dim3 grid;
  NL_TRY(bwd_grid(batch, heads, seq, a, grid));
  hipLaunchKernelGGL(flash_bwd_dkdv_kernel, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
  return nl_check_launch("nl_flash_attention_bwd_dkdv");
}

extern "C" size_t nl_flash_attention_bwd_ws_bytes(int batch, int heads, int seq) {
  if (batch <= 0 || heads <= 0 || seq <= 0) return 0;
  return (size_t)batch * heads * seq * sizeof(float);
}

extern "C" int nl_flash_attention_bwd(void* stream, int batch, int heads, int seq, int d_head, float scale,
                                      int causal, const nl_bf16* Q, nl_attn_stride sq, const nl_bf16* K,
                                      nl_attn_stride sk, const nl_bf16* V, nl_attn_stride sv, const nl_bf16* O,
                                      nl_attn_stride so, const nl_bf16* dO, nl_attn_stride sdo, const float* L,
                                      nl_bf16* dQ, nl_attn_stride sdq, nl_bf16* dK, nl_attn_stride sdk,
                                      nl_bf16* dV, nl_attn_stride sdv, void* ws) {
  NL_TRY(check_common(batch, heads, seq, d_head, causal));
  if (batch == 0 || heads == 0 || seq == 0) return NL_OK;
  if (!ws) return nl_set_error(NL_EINVAL, "flash: null workspace");
  if (((uintptr_t)ws & 15) != 0) return nl_set_error(NL_EALIGN, "flash: workspace not 16-byte aligned");
  float* D = static_cast<float*>(ws);
  NL_TRY(nl_flash_attention_bwd_preprocess(stream, batch, heads, seq, d_head, O, so, dO, sdo, D));
  NL_TRY(nl_flash_attention_bwd_dkdv(stream, batch, heads, seq, d_head, scale, causal, Q, sq, K, sk, V, sv, dO, sdo,
                                     L, D, dK, sdk, dV, sdv));
  NL_TRY(nl_flash_attention_bwd_dq(stream, batch, heads, seq, d_head, scale, causal, Q, sq, K, sk, V, sv, dO, sdo,
                                   L, D, dQ, sdq));
  return NL_OK;
}

// ---------------------------------------------------------------------------
// The backward without a caller workspace: D lives in a fixed device array.
// ---------------------------------------------------------------------------
// The array is a per-device global of the code object (each GPU holds its own
// copy, at its own address, until the process ends). Its host-side name is
// only a handle: kernels must be given the device address that
// hipGetSymbolAddress returns, looked up once per device and cached here.
static __device__ __align__(256) float scratch[NL_FLASH_BWD_NOALLOC_MAX_ROWS];

namespace nl {
namespace {
constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch_dev[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (first call per device
// resolves it with that device current).
int scratch_on_current_device(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return nl_set_error(NL_ELAUNCH, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return nl_set_error(NL_EUNSUPPORTED, "flash noalloc: device index >= 64");
  float* p = g_scratch_dev[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_dev[dev].load(std::memory_order_relaxed);
    if (!p) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !addr)
        return nl_set_error(NL_ELAUNCH, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
      p = static_cast<float*>(addr);
      g_scratch_dev[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return NL_OK;
}
}  // namespace
}  // namespace nl

extern "C" int nl_flash_attention_bwd_noalloc(void* stream, int batch, int heads, int seq, int d_head, float scale,
                                              int causal, const nl_bf16* Q, nl_attn_stride sq, const nl_bf16* K,
                                              nl_attn_stride sk, const nl_bf16* V, nl_attn_stride sv,
                                              const nl_bf16* O, nl_attn_stride so, const nl_bf16* dO,
                                              nl_attn_stride sdo, const float* L, nl_bf16* dQ, nl_attn_stride sdq,
                                              nl_bf16* dK, nl_attn_stride sdk, nl_bf16* dV, nl_attn_stride sdv) {
  NL_TRY(check_common(batch, heads, seq, d_head, causal));
  if (batch == 0 || heads == 0 || seq == 0) return NL_OK;
  if ((int64_t)batch * heads * seq > (int64_t)NL_FLASH_BWD_NOALLOC_MAX_ROWS)
    return nl_set_error(NL_EINVAL, "flash noalloc: batch*heads*seq exceeds NL_FLASH_BWD_NOALLOC_MAX_ROWS (" +
                                       std::to_string(NL_FLASH_BWD_NOALLOC_MAX_ROWS) + ")");
  float* D = nullptr;
  NL_TRY(scratch_on_current_device(&D));
  // D is written whole by the preprocess before dK/dV and dQ read it, so the
  // array needs no clearing between calls.
  return nl_flash_attention_bwd(stream, batch, heads, seq, d_head, scale, causal, Q, sq, K, sk, V, sv, O, so, dO, sdo,
                                L, dQ, sdq, dK, sdk, dV, sdv, D);
}
