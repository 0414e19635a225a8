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

struct FwdArgs {
  int S, causal;
  float scale_log2;
  Op q, k, v;
  OutOp o;
  float* L;
};

// Store a 32x32 transposed accumulator pair (d tiles 0/1) for the lane's row:
// lane (row, g) holds columns dt*32 + 8qq + 4g + t.
__device__ __forceinline__ void store_row64(uint16_t* rowp, const f32x16 acc[2], float mul, int g) {
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int col = dt * 32 + qq * 8 + 4 * g;
      *reinterpret_cast<u32x2*>(rowp + col) =
          u32x2{pack_bf16x2(acc[dt][4 * qq] * mul, acc[dt][4 * qq + 1] * mul),
                pack_bf16x2(acc[dt][4 * qq + 2] * mul, acc[dt][4 * qq + 3] * mul)};
    }
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void flash_fwd_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[2][kBlk * kD];
  const int S = a.S;
  const int nqt = (S + kRows - 1) / kRows;
  const int qt = nqt - 1 - (int)blockIdx.x;  // heaviest (latest) query tiles first
  const int h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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

  float m = -INFINITY, l = 0.f;
  f32x16 o[2];
  zero(o[0]);
  zero(o[1]);

  RowTile tk;
  TransTile tv;
  tk.load(a.k.at(b, h, 0), a.k.s.row, min(kBlk, S), tid);
  tv.load(a.v.at(b, h, 0), a.v.s.row, min(kBlk, S), tid);
  tk.store(sK[0], tid);
  tv.store(sVt[0], tid);
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    const int k0 = kb * kBlk;
    const bool more = kb + 1 < nkb;
    if (more) {
      tk.load(a.k.at(b, h, k0 + kBlk), a.k.s.row, min(kBlk, S - k0 - kBlk), tid);
      tv.load(a.v.at(b, h, k0 + kBlk), a.v.s.row, min(kBlk, S - k0 - kBlk), tid);
    }
    if (k0 < kend_w) {
      f32x16 s[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        zero(s[kt]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) s[kt] = mfma32(row_frag(sK[buf], kt * 32 + l32, ks * 2 + g), qf[ks], s[kt]);
      }
      const bool need_mask = (a.causal && k0 + kBlk - 1 > qw0) || (k0 + kBlk > S);
      float bm = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = s[kt][r] * a.scale_log2;
          if (need_mask) {
            const int key = k0 + kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
            if (key >= S || (a.causal && key > q)) x = -INFINITY;
          }
          s[kt][r] = x;
          bm = fmaxf(bm, x);
        }
      bm = fmaxf(bm, __shfl_xor(bm, 32, kWave));
      const float mn = fmaxf(m, bm);
      const float alpha = (m == -INFINITY) ? 0.f : fast_exp2(m - mn);
      float rs = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = (mn == -INFINITY) ? 0.f : fast_exp2(s[kt][r] - mn);
          s[kt][r] = p;
          rs += p;
        }
      l = l * alpha + rs;
      m = mn;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const bf16x8 pf = pack_frag(s[kt], hh);
#pragma unroll
          for (int dt = 0; dt < 2; ++dt)
            o[dt] = mfma32(trans_frag(sVt[buf], dt * 32 + l32, kt * 32 + hh * 16, g), pf, o[dt]);
        }
    }
    if (more) {
      tk.store(sK[buf ^ 1], tid);
      tv.store(sVt[buf ^ 1], tid);
    }
    __syncthreads();
  }

  const float lt = l + __shfl_xor(l, 32, kWave);
  if (qvalid) {
    const float inv = 1.f / lt;
    store_row64(a.o.at(b, h, q), o, inv, g);
    if (g == 0) a.L[((int64_t)b * gridDim.y + h) * S + q] = (m + fast_log2(lt)) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// backward preprocess: D = rowsum(dO o O)
// ---------------------------------------------------------------------------
struct PreArgs {
  int S, H, rows;
  Op o, dout;
  float* D;
};
__global__ __launch_bounds__(256) void flash_bwd_pre_kernel(PreArgs a) {
  // 8 lanes per row, 16 bytes each
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid >> 3;
  const int part = (int)(gid & 7);
  float acc = 0.f;
  if (row < a.rows) {
    const int s = (int)(row % a.S);
    const int bh = (int)(row / a.S);
    const int h = bh % a.H, b = bh / a.H;
    const u32x4 x = *reinterpret_cast<const u32x4*>(a.o.at(b, h, s) + part * 8);
    const u32x4 y = *reinterpret_cast<const u32x4*>(a.dout.at(b, h, s) + part * 8);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += bf16_lo(x[j]) * bf16_lo(y[j]) + bf16_hi(x[j]) * bf16_hi(y[j]);
  }
  acc += __shfl_xor(acc, 1, kWave);
  acc += __shfl_xor(acc, 2, kWave);
  acc += __shfl_xor(acc, 4, kWave);
  if (row < a.rows && part == 0) a.D[row] = acc;
}

struct BwdArgs {
  int S, causal;
  float scale, scale_log2;
  Op q, k, v, dout;
  const float* L;  // natural-log lse
  const float* D;
  OutOp dq, dk, dv;
};

// ---------------------------------------------------------------------------
// dK, dV: workgroup = 128 keys, streams 64-query blocks from the diagonal on
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void flash_bwd_dkdv_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sQ[2][kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sQt[2][kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sdO[2][kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sdOt[2][kBlk * kD];
  __shared__ __attribute__((aligned(16))) float sL[2][kBlk], sDv[2][kBlk];
  const int S = a.S;
  const int kt_idx = blockIdx.x;  // low key tiles see the most queries: launched first
  const int h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int kw0 = kt_idx * kRows + wave * 32;
  const int key = kw0 + l32;
  const bool kvalid = key < S;
  const int64_t lbase = ((int64_t)b * gridDim.y + h) * S;

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

  RowTile tq, tdo;
  TransTile tqt, tdot;
  float lv = 0.f, dv_ = 0.f;
  auto load_block = [&](int q0) {
    const int nv = min(kBlk, S - q0);
    tq.load(a.q.at(b, h, q0), a.q.s.row, nv, tid);
    tqt.load(a.q.at(b, h, q0), a.q.s.row, nv, tid);
    tdo.load(a.dout.at(b, h, q0), a.dout.s.row, nv, tid);
    tdot.load(a.dout.at(b, h, q0), a.dout.s.row, nv, tid);
    if (tid < kBlk) {
      lv = (tid < nv) ? a.L[lbase + q0 + tid] * kLog2e : INFINITY;  // +inf -> P = 0 for padding rows
      dv_ = (tid < nv) ? a.D[lbase + q0 + tid] : 0.f;
    }
  };
  auto store_block = [&](int buf) {
    tq.store(sQ[buf], tid);
    tqt.store(sQt[buf], tid);
    tdo.store(sdO[buf], tid);
    tdot.store(sdOt[buf], tid);
    if (tid < kBlk) {
      sL[buf][tid] = lv;
      sDv[buf][tid] = dv_;
    }
  };
  if (nqb > 0) {
    load_block(qstart);
    store_block(0);
  }
  __syncthreads();

  for (int qb = 0; qb < nqb; ++qb) {
    const int buf = qb & 1;
    const int q0 = qstart + qb * kBlk;
    const bool more = qb + 1 < nqb;
    if (more) load_block(q0 + kBlk);
    // this wave's keys see queries >= kw0 only (causal)
    if (!a.causal || q0 + kBlk - 1 >= kw0) {
      const bool need_mask = (a.causal && q0 < kw0 + 31) || (q0 + kBlk > S);
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        f32x16 s, dp;
        zero(s);
        zero(dp);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          s = mfma32(row_frag(sQ[buf], qt * 32 + l32, ks * 2 + g), kf[ks], s);
          dp = mfma32(row_frag(sdO[buf], qt * 32 + l32, ks * 2 + g), vf[ks], dp);
        }
        // lane (key, g) holds query rows qt*32 + 8qq + 4g + t
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int qr = qt * 32 + qq * 8 + 4 * g;
          const f32x4 L4 = *reinterpret_cast<const f32x4*>(&sL[buf][qr]);
          const f32x4 D4 = *reinterpret_cast<const f32x4*>(&sDv[buf][qr]);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int r = 4 * qq + t;
            float p = fast_exp2(__builtin_fmaf(s[r], a.scale_log2, -L4[t]));
            if (need_mask) {
              const int qi = q0 + qr + t;
              if (qi >= S || (a.causal && qi < key)) p = 0.f;
            }
            s[r] = p;
            dp[r] = p * (dp[r] - D4[t]);
          }
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const bf16x8 pf = pack_frag(s, hh);
          const bf16x8 dsf = pack_frag(dp, hh);
#pragma unroll
          for (int dt = 0; dt < 2; ++dt) {
            dv[dt] = mfma32(trans_frag(sdOt[buf], dt * 32 + l32, qt * 32 + hh * 16, g), pf, dv[dt]);
            dk[dt] = mfma32(trans_frag(sQt[buf], dt * 32 + l32, qt * 32 + hh * 16, g), dsf, dk[dt]);
          }
        }
      }
    }
    if (more) store_block(buf ^ 1);
    __syncthreads();
  }
  if (kvalid) {
    store_row64(a.dk.at(b, h, key), dk, a.scale, g);
    store_row64(a.dv.at(b, h, key), dv, 1.f, g);
  }
}

// ---------------------------------------------------------------------------
// dQ: workgroup = 128 queries, streams 64-key blocks up to the diagonal
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void flash_bwd_dq_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][kBlk * kD];
  __shared__ __attribute__((aligned(16))) uint16_t sKt[2][kBlk * kD];
  const int S = a.S;
  const int nqt = (S + kRows - 1) / kRows;
  const int qt = nqt - 1 - (int)blockIdx.x;
  const int h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int qw0 = qt * kRows + wave * 32;
  const int q = qw0 + l32;
  const bool qvalid = q < S;
  const int64_t lbase = ((int64_t)b * gridDim.y + h) * S;

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
  const float Lq = qvalid ? a.L[lbase + q] * kLog2e : INFINITY;
  const float Dq = qvalid ? a.D[lbase + q] : 0.f;

  const int kend_wg = a.causal ? min(S, qt * kRows + kRows) : S;
  const int kend_w = a.causal ? min(S, qw0 + 32) : S;
  const int nkb = (kend_wg + kBlk - 1) / kBlk;

  f32x16 dq[2];
  zero(dq[0]);
  zero(dq[1]);

  RowTile tk, tv;
  TransTile tkt;
  tk.load(a.k.at(b, h, 0), a.k.s.row, min(kBlk, S), tid);
  tv.load(a.v.at(b, h, 0), a.v.s.row, min(kBlk, S), tid);
  tkt.load(a.k.at(b, h, 0), a.k.s.row, min(kBlk, S), tid);
  tk.store(sK[0], tid);
  tv.store(sV[0], tid);
  tkt.store(sKt[0], tid);
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    const int k0 = kb * kBlk;
    const bool more = kb + 1 < nkb;
    if (more) {
      const int nv = min(kBlk, S - k0 - kBlk);
      tk.load(a.k.at(b, h, k0 + kBlk), a.k.s.row, nv, tid);
      tv.load(a.v.at(b, h, k0 + kBlk), a.v.s.row, nv, tid);
      tkt.load(a.k.at(b, h, k0 + kBlk), a.k.s.row, nv, tid);
    }
    if (k0 < kend_w) {
      const bool need_mask = (a.causal && k0 + kBlk - 1 > qw0) || (k0 + kBlk > S);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        f32x16 s, dp;
        zero(s);
        zero(dp);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          s = mfma32(row_frag(sK[buf], kt * 32 + l32, ks * 2 + g), qf[ks], s);
          dp = mfma32(row_frag(sV[buf], kt * 32 + l32, ks * 2 + g), df[ks], dp);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float p = fast_exp2(__builtin_fmaf(s[r], a.scale_log2, -Lq));
          if (need_mask) {
            const int key = k0 + kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
            if (key >= S || (a.causal && key > q)) p = 0.f;
          }
          dp[r] = p * (dp[r] - Dq);
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const bf16x8 dsf = pack_frag(dp, hh);
#pragma unroll
          for (int dt = 0; dt < 2; ++dt)
            dq[dt] = mfma32(trans_frag(sKt[buf], dt * 32 + l32, kt * 32 + hh * 16, g), dsf, dq[dt]);
        }
      }
    }
    if (more) {
      tk.store(sK[buf ^ 1], tid);
      tv.store(sV[buf ^ 1], tid);
      tkt.store(sKt[buf ^ 1], tid);
    }
    __syncthreads();
  }
  if (qvalid) store_row64(a.dq.at(b, h, q), dq, a.scale, g);
}

// ---------------------------------------------------------------------------
// host-side validation
// ---------------------------------------------------------------------------
bool stride_ok(const nl_attn_stride& s) { return ((s.batch | s.head | s.row) & 7) == 0 && s.row >= 64; }

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
  FwdArgs a;
  a.S = seq;
  a.causal = causal;
  a.scale_log2 = scale * kLog2e;
  a.q = Op{Q, sq};
  a.k = Op{K, sk};
  a.v = Op{V, sv};
  a.o = OutOp{O, so};
  a.L = L;
  dim3 grid((seq + kRows - 1) / kRows, heads, batch);
  hipLaunchKernelGGL(flash_fwd_kernel, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
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
  a.rows = batch * heads * seq;
  a.o = Op{O, so};
  a.dout = Op{dO, sdo};
  a.D = D;
  const int64_t threads = (int64_t)a.rows * 8;
  hipLaunchKernelGGL(flash_bwd_pre_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, a);
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
  dim3 grid((seq + kRows - 1) / kRows, heads, batch);
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
  dim3 grid((seq + kRows - 1) / kRows, heads, batch);
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
