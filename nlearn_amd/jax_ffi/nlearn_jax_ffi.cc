// nlearn_jax_ffi.cc — XLA FFI handlers that bind the reference's jax.ffi
// targets to libnlearn_hip.so on JAX-ROCm.
//
// Not built in this repository: JAX and the XLA FFI headers are not installed
// here. On a JAX-ROCm install:
//   hipcc --offload-arch=gfx950 -std=c++17 -shared -fPIC \
//         -I"$(python -c 'import jax.ffi; print(jax.ffi.include_dir())')" -Iinclude \
//         nlearn_amd/jax_ffi/nlearn_jax_ffi.cc -Lnlearn_amd -lnlearn_hip -o libnlearn_jax_ffi.so
// and register the handlers with nlearn_amd/jax_ffi/register.py.
//
// Operand lists are those of the reference's ffi_call sites:
//   flash_attention_fwd       (Q, K, V)            -> (O, L)     attention.py:82-91
//   flash_attention_bwd_dq    (Q, K, V, dO, L, D)  -> dQ         attention.py:117-121
//   flash_attention_bwd_dkdv  (Q, K, V, dO, L, D)  -> (dK, dV)   attention.py:122-127
//   gemm                      (A, B)               -> C          gemm.py:32-40
//   gemm_nt                   (dC, B)              -> dA = dC B^T  (gemm.py:74, no transpose)
//   gemm_tn                   (A, dC)              -> dB = A^T dC  (gemm.py:75, no transpose)
//   ce_fwd                    (logits, targets)    -> (loss, lse)  cross_entropy.py:28-36
//   ce_bwd                    (logits, targets, lse) -> dlogits    cross_entropy.py:39-46
//   ce_fwd_bwd                (logits, targets)    -> (loss, lse, dlogits), one pass;
//                             bind with input_output_aliases={0: 2} to write dlogits
//                             over the logits (cross_entropy.py:55-65 fused)
// Shapes carry everything (no attributes), as in the reference: scale =
// 1/sqrt(d) for flash, 1/M for the CE gradient.
//
// Boundary dtype: bf16 tensors where the reference passes f32 after its
// astype(jnp.float32) casts (attention.py:97,104,115; cross_entropy.py:76);
// those casts become astype(jnp.bfloat16), and the results declared for O,
// dQ, dK, dV and dlogits (attention.py:88,119,124-125; cross_entropy.py:44)
// become jnp.bfloat16 with them. L, D (attention.py:116, reduced from f32
// upcasts of dO and O), loss, lse and the GEMM's C stay f32.
// register.py's CALL_SITES lists every operand and result dtype with its
// reference line; the bindings at the end of this file must equal it.
//
// Alignment: the kernels need 16-byte row starts for the GEMM (ld % 8 == 0).
// The gemm handlers take dense XLA buffers, so K and N must be multiples of 8:
// the reference's _gemm_padded (gemm.py:47-58) pads K to 64 and N to 32, which
// satisfies it; keep that padding at the three GEMM call sites. The flash and
// CE handlers have no such requirement (d = 64 rows are 128 bytes; the CE
// peels unaligned row heads).
#include <cmath>
#include <cstdint>
#include <string>

#include <hip/hip_runtime.h>

#include "nlearn_hip.h"
#include "xla/ffi/api/ffi.h"

namespace ffi = xla::ffi;

namespace {

ffi::Error status(int rc) {
  if (rc == NL_OK) return ffi::Error::Success();
  return ffi::Error(rc == NL_ELAUNCH ? ffi::ErrorCode::kInternal : ffi::ErrorCode::kInvalidArgument,
                    std::string(nl_last_error()));
}

ffi::Error bad(const char* msg) { return ffi::Error(ffi::ErrorCode::kInvalidArgument, msg); }

template <class B>
const nl_bf16* bf(const B& b) { return static_cast<const nl_bf16*>(b.untyped_data()); }
template <class B>
nl_bf16* bf_out(B& b) { return static_cast<nl_bf16*>(b->untyped_data()); }
template <class B>
const float* f32(const B& b) { return static_cast<const float*>(b.untyped_data()); }
template <class B>
float* f32_out(B& b) { return static_cast<float*>(b->untyped_data()); }

// (n, s, d) contiguous: one "batch" of n heads, element (b, 0, t, c) at b*s*d + t*d + c
nl_attn_stride dense3(int64_t s, int64_t d) { return nl_attn_stride{s * d, 0, d}; }

// ---- flash attention ------------------------------------------------------

ffi::Error FlashFwd(hipStream_t st, ffi::Buffer<ffi::BF16> q, ffi::Buffer<ffi::BF16> k, ffi::Buffer<ffi::BF16> v,
                    ffi::ResultBuffer<ffi::BF16> o, ffi::ResultBuffer<ffi::F32> l) {
  auto dm = q.dimensions();
  if (dm.size() != 3) return bad("flash_attention_fwd: Q must be (n, s, d)");
  const int n = (int)dm[0], s = (int)dm[1], d = (int)dm[2];
  const nl_attn_stride sd = dense3(s, d);
  return status(nl_flash_attention_fwd(st, n, 1, s, d, 1.0f / std::sqrt((float)d), 1, bf(q), sd, bf(k), sd, bf(v),
                                       sd, bf_out(o), sd, f32_out(l)));
}

ffi::Error FlashBwdDq(hipStream_t st, ffi::Buffer<ffi::BF16> q, ffi::Buffer<ffi::BF16> k, ffi::Buffer<ffi::BF16> v,
                      ffi::Buffer<ffi::BF16> dout, ffi::Buffer<ffi::F32> l, ffi::Buffer<ffi::F32> dd,
                      ffi::ResultBuffer<ffi::BF16> dq) {
  auto dm = q.dimensions();
  if (dm.size() != 3) return bad("flash_attention_bwd_dq: Q must be (n, s, d)");
  const int n = (int)dm[0], s = (int)dm[1], d = (int)dm[2];
  const nl_attn_stride sd = dense3(s, d);
  return status(nl_flash_attention_bwd_dq(st, n, 1, s, d, 1.0f / std::sqrt((float)d), 1, bf(q), sd, bf(k), sd, bf(v),
                                          sd, bf(dout), sd, f32(l), f32(dd), bf_out(dq), sd));
}

ffi::Error FlashBwdDkdv(hipStream_t st, ffi::Buffer<ffi::BF16> q, ffi::Buffer<ffi::BF16> k,
                        ffi::Buffer<ffi::BF16> v, ffi::Buffer<ffi::BF16> dout, ffi::Buffer<ffi::F32> l,
                        ffi::Buffer<ffi::F32> dd, ffi::ResultBuffer<ffi::BF16> dk, ffi::ResultBuffer<ffi::BF16> dv) {
  auto dm = q.dimensions();
  if (dm.size() != 3) return bad("flash_attention_bwd_dkdv: Q must be (n, s, d)");
  const int n = (int)dm[0], s = (int)dm[1], d = (int)dm[2];
  const nl_attn_stride sd = dense3(s, d);
  return status(nl_flash_attention_bwd_dkdv(st, n, 1, s, d, 1.0f / std::sqrt((float)d), 1, bf(q), sd, bf(k), sd,
                                            bf(v), sd, bf(dout), sd, f32(l), f32(dd), bf_out(dk), sd, bf_out(dv),
                                            sd));
}

// ---- GEMM -------------------------------------------------------------------

// C (M, N) f32 = A (M, K) . B (K, N)
ffi::Error Gemm(hipStream_t st, ffi::Buffer<ffi::BF16> a, ffi::Buffer<ffi::BF16> b, ffi::ResultBuffer<ffi::F32> c) {
  if (a.dimensions().size() != 2 || b.dimensions().size() != 2) return bad("gemm: A and B must be 2-D");
  const int64_t M = a.dimensions()[0], K = a.dimensions()[1], N = b.dimensions()[1];
  if (b.dimensions()[0] != K) return bad("gemm: inner dimensions differ");
  return status(nl_gemm(st, NL_OP_N, NL_OP_N, (int)M, (int)N, (int)K, 1.0f, bf(a), K, bf(b), N, 0.0f, f32_out(c),
                        NL_DTYPE_F32, N, nullptr));
}

// dA (M, K) f32 = dC (M, N) . B^T, with B stored (K, N)
ffi::Error GemmNT(hipStream_t st, ffi::Buffer<ffi::BF16> dc, ffi::Buffer<ffi::BF16> b,
                  ffi::ResultBuffer<ffi::F32> da) {
  if (dc.dimensions().size() != 2 || b.dimensions().size() != 2) return bad("gemm_nt: operands must be 2-D");
  const int64_t M = dc.dimensions()[0], N = dc.dimensions()[1], K = b.dimensions()[0];
  if (b.dimensions()[1] != N) return bad("gemm_nt: dC and B disagree on N");
  return status(nl_gemm(st, NL_OP_N, NL_OP_T, (int)M, (int)K, (int)N, 1.0f, bf(dc), N, bf(b), N, 0.0f, f32_out(da),
                        NL_DTYPE_F32, K, nullptr));
}

// dB (K, N) f32 = A^T . dC, with A stored (M, K) and dC (M, N)
ffi::Error GemmTN(hipStream_t st, ffi::Buffer<ffi::BF16> a, ffi::Buffer<ffi::BF16> dc,
                  ffi::ResultBuffer<ffi::F32> db) {
  if (a.dimensions().size() != 2 || dc.dimensions().size() != 2) return bad("gemm_tn: operands must be 2-D");
  const int64_t M = a.dimensions()[0], K = a.dimensions()[1], N = dc.dimensions()[1];
  if (dc.dimensions()[0] != M) return bad("gemm_tn: A and dC disagree on M");
  return status(nl_gemm(st, NL_OP_T, NL_OP_N, (int)K, (int)N, (int)M, 1.0f, bf(a), K, bf(dc), N, 0.0f, f32_out(db),
                        NL_DTYPE_F32, N, nullptr));
}

// ---- cross-entropy ------------------------------------------------------------

ffi::Error CeFwd(hipStream_t st, ffi::Buffer<ffi::BF16> logits, ffi::Buffer<ffi::S32> targets,
                 ffi::ResultBuffer<ffi::F32> loss, ffi::ResultBuffer<ffi::F32> lse) {
  if (logits.dimensions().size() != 2) return bad("ce_fwd: logits must be (M, V)");
  const int64_t M = logits.dimensions()[0], V = logits.dimensions()[1];
  return status(nl_ce_fwd(st, (int)M, (int)V, bf(logits), V, static_cast<const int32_t*>(targets.untyped_data()),
                          f32_out(loss), f32_out(lse)));
}

// dlogits = (softmax - onehot) / M, as the reference's ce_bwd returns it
ffi::Error CeBwd(hipStream_t st, ffi::Buffer<ffi::BF16> logits, ffi::Buffer<ffi::S32> targets,
                 ffi::Buffer<ffi::F32> lse, ffi::ResultBuffer<ffi::BF16> dlogits) {
  if (logits.dimensions().size() != 2) return bad("ce_bwd: logits must be (M, V)");
  const int64_t M = logits.dimensions()[0], V = logits.dimensions()[1];
  return status(nl_ce_bwd(st, (int)M, (int)V, bf(logits), V, static_cast<const int32_t*>(targets.untyped_data()),
                          f32(lse), M > 0 ? 1.0f / (float)M : 0.0f, bf_out(dlogits), V));
}

// loss, lse and dlogits in one read of the logits (dlogits may alias them)
ffi::Error CeFwdBwd(hipStream_t st, ffi::Buffer<ffi::BF16> logits, ffi::Buffer<ffi::S32> targets,
                    ffi::ResultBuffer<ffi::F32> loss, ffi::ResultBuffer<ffi::F32> lse,
                    ffi::ResultBuffer<ffi::BF16> dlogits) {
  if (logits.dimensions().size() != 2) return bad("ce_fwd_bwd: logits must be (M, V)");
  const int64_t M = logits.dimensions()[0], V = logits.dimensions()[1];
  return status(nl_ce_fwd_bwd(st, (int)M, (int)V, bf(logits), V,
                              static_cast<const int32_t*>(targets.untyped_data()), f32_out(loss), f32_out(lse),
                              M > 0 ? 1.0f / (float)M : 0.0f, bf_out(dlogits), V));
}

}  // namespace

// ---- handler symbols (the names register.py looks up) -------------------------

#define NL_BIND ffi::Ffi::Bind().Ctx<ffi::PlatformStream<hipStream_t>>()
#define NL_ARG(T) .Arg<ffi::Buffer<ffi::T>>()
#define NL_RET(T) .Ret<ffi::Buffer<ffi::T>>()

XLA_FFI_DEFINE_HANDLER_SYMBOL(nl_flash_attention_fwd_ffi, FlashFwd,
                              NL_BIND NL_ARG(BF16) NL_ARG(BF16) NL_ARG(BF16) NL_RET(BF16) NL_RET(F32));
XLA_FFI_DEFINE_HANDLER_SYMBOL(nl_flash_attention_bwd_dq_ffi, FlashBwdDq,
                              NL_BIND NL_ARG(BF16) NL_ARG(BF16) NL_ARG(BF16) NL_ARG(BF16) NL_ARG(F32) NL_ARG(F32)
                                  NL_RET(BF16));
XLA_FFI_DEFINE_HANDLER_SYMBOL(nl_flash_attention_bwd_dkdv_ffi, FlashBwdDkdv,
                              NL_BIND NL_ARG(BF16) NL_ARG(BF16) NL_ARG(BF16) NL_ARG(BF16) NL_ARG(F32) NL_ARG(F32)
                                  NL_RET(BF16) NL_RET(BF16));
XLA_FFI_DEFINE_HANDLER_SYMBOL(nl_gemm_ffi, Gemm, NL_BIND NL_ARG(BF16) NL_ARG(BF16) NL_RET(F32));
XLA_FFI_DEFINE_HANDLER_SYMBOL(nl_gemm_nt_ffi, GemmNT, NL_BIND NL_ARG(BF16) NL_ARG(BF16) NL_RET(F32));
XLA_FFI_DEFINE_HANDLER_SYMBOL(nl_gemm_tn_ffi, GemmTN, NL_BIND NL_ARG(BF16) NL_ARG(BF16) NL_RET(F32));
XLA_FFI_DEFINE_HANDLER_SYMBOL(nl_ce_fwd_ffi, CeFwd, NL_BIND NL_ARG(BF16) NL_ARG(S32) NL_RET(F32) NL_RET(F32));
XLA_FFI_DEFINE_HANDLER_SYMBOL(nl_ce_bwd_ffi, CeBwd,
                              NL_BIND NL_ARG(BF16) NL_ARG(S32) NL_ARG(F32) NL_RET(BF16));
XLA_FFI_DEFINE_HANDLER_SYMBOL(nl_ce_fwd_bwd_ffi, CeFwdBwd,
                              NL_BIND NL_ARG(BF16) NL_ARG(S32) NL_RET(F32) NL_RET(F32) NL_RET(BF16));
