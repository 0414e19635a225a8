/*
 * nlearn_hip.h — C ABI of the MI355X (gfx950) kernels behind nlearn's three
 * training hot paths: causal FlashAttention (forward + recompute backward), the
 * bf16 GEMM used by `linear`, and the fused softmax cross-entropy.
 *
 * Conventions shared by every entry point
 *   - Plain C types only. `stream` is a hipStream_t passed as void* (NULL = the
 *     default stream). Every call is stream-ordered and asynchronous: no host
 *     synchronisation, no device allocation, no global mutable state.
 *   - Tensors are device pointers. bf16 values are raw IEEE bfloat16 bit
 *     patterns (nl_bf16 = uint16_t). All arithmetic inside the kernels is fp32.
 *   - Matrices are row-major with an explicit leading dimension (elements
 *     between consecutive rows). Row-major dense tensors pass ld = #columns.
 *   - Return value: NL_OK (0) on success, otherwise an NL_E* code. Argument
 *     errors are detected on the host before anything is launched; launch
 *     failures report hipGetLastError. nl_last_error() gives a message for the
 *     most recent failure on the calling thread.
 *
 * Reference interfaces replaced (paths relative to the nlearn repository):
 *   jax.ffi target "flash_attention_fwd"       nlearn/attention.py:82-91
 *   jax.ffi target "flash_attention_bwd_dq"    nlearn/attention.py:117-121
 *   jax.ffi target "flash_attention_bwd_dkdv"  nlearn/attention.py:122-127
 *   XLA D = sum(dO*O, -1)                      nlearn/attention.py:116
 *   jax.ffi target "gemm" + _gemm_padded       nlearn/kernels/gemm.py:32-58
 *   _gemm_bwd transposes                       nlearn/kernels/gemm.py:71-76
 *   jax.ffi target "ce_fwd"                    nlearn/kernels/cross_entropy.py:28-36
 *   jax.ffi target "ce_bwd"                    nlearn/kernels/cross_entropy.py:39-46
 *   loss.mean() / g * dlogits                  nlearn/kernels/cross_entropy.py:51,65
 */
#ifndef NLEARN_HIP_H
#define NLEARN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t nl_bf16;

/* ---- status codes ------------------------------------------------------- */
#define NL_OK           0
#define NL_EINVAL       1  /* bad shape, size or enum argument              */
#define NL_EALIGN       2  /* pointer or leading dimension misaligned       */
#define NL_EUNSUPPORTED 3  /* valid request this build does not implement   */
#define NL_ELAUNCH      4  /* kernel launch failed (hipGetLastError)        */

const char* nl_strerror(int status);
/* Message of the most recent failing call on this thread ("" if none). */
const char* nl_last_error(void);
/* Library version string, e.g. "nlearn_hip 0.1 gfx950". */
const char* nl_version(void);

/* ======================================================================== */
/* GEMM                                                                      */
/* ======================================================================== */
/*
 * C[M,N] = alpha * s * op(A)[M,K] . op(B)[K,N] + beta * C
 *   s = *alpha_dev if alpha_dev != NULL, else 1 (a device-side scale factor,
 *       used to fold an upstream cotangent into the product without a sync).
 *   op(A) = A   stored [M][lda] (opA = NL_OP_N)   or
 *         = A^T with A stored [K][lda] (opA = NL_OP_T);
 *   op(B) = B   stored [K][ldb] (opB = NL_OP_N)   or
 *         = B^T with B stored [N][ldb] (opB = NL_OP_T).
 * A, B are bf16; the product accumulates in fp32; C is fp32 or bf16 (RNE).
 * beta == 0 never reads C. Tails in M, N and K are handled in-kernel (no host
 * padding). Requirements: A, B, C 16-byte aligned; lda, ldb, ldc multiples of
 * 8; M, N, K >= 0 (an empty product with K == 0 writes beta*C).
 *
 * Replaces: gemm(A,B) -> f32 C (gemm.py:32-40, 61-64) with opA=opB=N;
 *   dA = dC . B^T  (gemm.py:74) with opA=N, opB=T, no materialised transpose;
 *   dB = A^T . dC  (gemm.py:75) with opA=T, opB=N, no materialised transpose.
 */
#define NL_OP_N 0
#define NL_OP_T 1
#define NL_DTYPE_F32  0
#define NL_DTYPE_BF16 1

int nl_gemm(void* stream, int opA, int opB, int M, int N, int K,
            float alpha, const nl_bf16* A, int64_t lda,
            const nl_bf16* B, int64_t ldb,
            float beta, void* C, int c_dtype, int64_t ldc,
            const float* alpha_dev);

/* nl_gemm with a caller-owned device workspace. Products with a small output
 * and a long reduction (the weight gradient X^T.dY reduces over all tokens)
 * split K across workgroups into fp32 partials that a second kernel sums in a
 * fixed order (deterministic). nl_gemm_ws_bytes() gives the size this build
 * wants for a shape (0 = no split); a NULL or smaller workspace just disables
 * the split. Same result contract as nl_gemm. */
size_t nl_gemm_ws_bytes(int opA, int opB, int M, int N, int K);
int nl_gemm_ex(void* stream, int opA, int opB, int M, int N, int K,
               float alpha, const nl_bf16* A, int64_t lda,
               const nl_bf16* B, int64_t ldb,
               float beta, void* C, int c_dtype, int64_t ldc,
               const float* alpha_dev, void* ws, size_t ws_bytes);

/* nl_gemm_ex with a fused output stage applied to v = alpha * s * op(A).op(B)
 * before C is written (and, when K is split, after the ordered reduction):
 *   NL_EPI_NONE       C = v + beta * C                       (= nl_gemm_ex)
 *   NL_EPI_BIAS       C = v + bias[n] + beta * C
 *   NL_EPI_BIAS_GELU  u = bf16(v + bias[n]); aux[m][n] = u; C = gelu_tanh(u)
 *   NL_EPI_DGELU      C = v * gelu_tanh'(aux[m][n])          (aux = the u saved above)
 * bias is fp32 [N], 16-byte aligned; aux is bf16 [M][ldaux], 16-byte aligned,
 * ldaux >= N and a multiple of 8; the GELU forms need beta == 0.
 * gelu_tanh(u) = u/2 (1 + tanh(sqrt(2/pi) (u + 0.044715 u^3))).
 *
 * Replaces the XLA-fused elementwise work around linear() in the FFN,
 * model.py:266-277 (linear -> activation -> linear) and its autodiff; the
 * benchmark layout uses the tanh-GELU with biases b1, b2 in place of the
 * current SwiGLU gate. */
#define NL_EPI_NONE      0
#define NL_EPI_BIAS      1
#define NL_EPI_BIAS_GELU 2
#define NL_EPI_DGELU     3
int nl_gemm_fused(void* stream, int opA, int opB, int M, int N, int K,
                  float alpha, const nl_bf16* A, int64_t lda,
                  const nl_bf16* B, int64_t ldb,
                  float beta, void* C, int c_dtype, int64_t ldc,
                  const float* alpha_dev, int epi, const float* bias,
                  nl_bf16* aux, int64_t ldaux, void* ws, size_t ws_bytes);

/* ======================================================================== */
/* Causal FlashAttention (head dim 64)                                        */
/* ======================================================================== */
/*
 * Strided layout of one attention operand: element (b, h, s, d) lives at
 *   base + b*batch + h*head + s*row + d        (d is contiguous).
 * The reference's contiguous (n, s, d) tensors are batch = s*d, head = 0 with
 * heads = 1 (or any equivalent split of n). The strided form lets a caller
 * hand over the fused QKV projection output [bs, s, 3*H*64] directly, with no
 * head-folding transposes (model.py:173-198 does them in XLA).
 * L and D are always dense fp32 [batch][heads][seq].
 */
typedef struct nl_attn_stride {
  int64_t batch;
  int64_t head;
  int64_t row;
} nl_attn_stride;

/*
 * O = softmax(scale * Q K^T + causal mask) V,  L = logsumexp row (natural log).
 * Requires d_head == 64, seq >= 0 (any length; tails masked), strides multiples
 * of 8 elements with row >= 64, and 16-byte aligned bases. causal = 1 is the
 * reference's causal mask (flash_attention.metal:107); causal = 0 attends to
 * every key.
 * Replaces "flash_attention_fwd" (attention.py:82-91, flash_attention.metal:55-146).
 */
int nl_flash_attention_fwd(void* stream, int batch, int heads, int seq, int d_head,
                           float scale, int causal,
                           const nl_bf16* Q, nl_attn_stride sq,
                           const nl_bf16* K, nl_attn_stride sk,
                           const nl_bf16* V, nl_attn_stride sv,
                           nl_bf16* O, nl_attn_stride so,
                           float* L);

/* D[b,h,s] = sum_d dO * O  (fp32).  Replaces attention.py:116. */
int nl_flash_attention_bwd_preprocess(void* stream, int batch, int heads, int seq,
                                      int d_head,
                                      const nl_bf16* O, nl_attn_stride so,
                                      const nl_bf16* dO, nl_attn_stride sdo,
                                      float* D);

/* dQ = scale * dS K with dS = P o (dP - D), P recomputed from L.
 * Replaces "flash_attention_bwd_dq" (attention.py:117-121,
 * flash_attention.metal:168-243). */
int nl_flash_attention_bwd_dq(void* stream, int batch, int heads, int seq, int d_head,
                              float scale, int causal,
                              const nl_bf16* Q, nl_attn_stride sq,
                              const nl_bf16* K, nl_attn_stride sk,
                              const nl_bf16* V, nl_attn_stride sv,
                              const nl_bf16* dO, nl_attn_stride sdo,
                              const float* L, const float* D,
                              nl_bf16* dQ, nl_attn_stride sdq);

/* dV = P^T dO, dK = scale * dS^T Q.
 * Replaces "flash_attention_bwd_dkdv" (attention.py:122-127,
 * flash_attention.metal:265-347). */
int nl_flash_attention_bwd_dkdv(void* stream, int batch, int heads, int seq, int d_head,
                                float scale, int causal,
                                const nl_bf16* Q, nl_attn_stride sq,
                                const nl_bf16* K, nl_attn_stride sk,
                                const nl_bf16* V, nl_attn_stride sv,
                                const nl_bf16* dO, nl_attn_stride sdo,
                                const float* L, const float* D,
                                nl_bf16* dK, nl_attn_stride sdk,
                                nl_bf16* dV, nl_attn_stride sdv);

/* Whole backward (preprocess + dK/dV + dQ) in one call. `ws` is a caller-owned
 * device workspace of nl_flash_attention_bwd_ws_bytes() bytes (holds D).
 * Replaces _flash_bwd_rule (attention.py:111-128). */
size_t nl_flash_attention_bwd_ws_bytes(int batch, int heads, int seq);
int nl_flash_attention_bwd(void* stream, int batch, int heads, int seq, int d_head,
                           float scale, int causal,
                           const nl_bf16* Q, nl_attn_stride sq,
                           const nl_bf16* K, nl_attn_stride sk,
                           const nl_bf16* V, nl_attn_stride sv,
                           const nl_bf16* O, nl_attn_stride so,
                           const nl_bf16* dO, nl_attn_stride sdo,
                           const float* L,
                           nl_bf16* dQ, nl_attn_stride sdq,
                           nl_bf16* dK, nl_attn_stride sdk,
                           nl_bf16* dV, nl_attn_stride sdv,
                           void* ws);

/* nl_flash_attention_bwd without a workspace argument: D lives in a fixed
 * device array inside this library (NL_FLASH_BWD_NOALLOC_MAX_ROWS floats,
 * 8 MiB, held by every GPU the library runs on until the process ends), so the
 * call allocates nothing and needs nothing from the caller beyond inputs and
 * outputs. It has no counterpart in the reference: it is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). batch*heads*seq above the maximum returns
 * NL_EINVAL before anything is launched. The stream must belong to the
 * current device; the first call on a device resolves the array's address
 * there (make it before any graph capture). All calls on one GPU share the
 * array: calls that overlap in time on one GPU (two streams, two threads)
 * race on D and must be serialised by the caller. Results are those of
 * nl_flash_attention_bwd, bit for bit. */
#define NL_FLASH_BWD_NOALLOC_MAX_ROWS 2097152
int nl_flash_attention_bwd_noalloc(void* stream, int batch, int heads, int seq, int d_head,
                                   float scale, int causal,
                                   const nl_bf16* Q, nl_attn_stride sq,
                                   const nl_bf16* K, nl_attn_stride sk,
                                   const nl_bf16* V, nl_attn_stride sv,
                                   const nl_bf16* O, nl_attn_stride so,
                                   const nl_bf16* dO, nl_attn_stride sdo,
                                   const float* L,
                                   nl_bf16* dQ, nl_attn_stride sdq,
                                   nl_bf16* dK, nl_attn_stride sdk,
                                   nl_bf16* dV, nl_attn_stride sdv);

/* ======================================================================== */
/* Softmax cross-entropy                                                      */
/* ======================================================================== */
/*
 * logits: bf16 [M][ld_logits] (V valid columns); targets: int32 [M].
 * A target outside [0, V) yields loss = NaN for that row (the reference kernel
 * has no check and reads out of bounds, cross_entropy.metal:66).
 */

/* loss[m] = lse[m] - logits[m, t[m]],  lse[m] = logsumexp(logits[m]).
 * Replaces "ce_fwd" (cross_entropy.py:28-36, cross_entropy.metal:38-68). */
int nl_ce_fwd(void* stream, int M, int V,
              const nl_bf16* logits, int64_t ld_logits, const int32_t* targets,
              float* loss, float* lse);

/* dlogits[m,v] = (exp(logits[m,v] - lse[m]) - [v == t[m]]) * scale  (bf16).
 * The reference uses scale = 1/M. Replaces "ce_bwd" (cross_entropy.py:39-46,
 * cross_entropy.metal:81-97). */
int nl_ce_bwd(void* stream, int M, int V,
              const nl_bf16* logits, int64_t ld_logits, const int32_t* targets,
              const float* lse, float scale,
              nl_bf16* dlogits, int64_t ld_dlogits);

/* Single pass over the logits: loss, lse and dlogits together. dlogits may
 * alias logits (then ld_dlogits must equal ld_logits) and is written in place.
 * Fuses ce_fwd + ce_bwd (cross_entropy.py:55-65). */
int nl_ce_fwd_bwd(void* stream, int M, int V,
                  const nl_bf16* logits, int64_t ld_logits, const int32_t* targets,
                  float* loss, float* lse, float scale,
                  nl_bf16* dlogits, int64_t ld_dlogits);

/* Fused LM head + cross-entropy: the CE of logits = X[M][D] . W[D][V] without
 * the (M, V) logits in memory. Replaces linear_cross_entropy
 * (cross_entropy.py:84-170, selected by NLEARN_FUSED_LMHEAD=1 in
 * train.py:24-28,279-283), which chunks the vocabulary and recomputes each
 * chunk's logits in the backward. X and W are bf16, row-major, 16-byte aligned
 * with ldx, ldw multiples of 8; the logits both entry points work from are
 * l = bf16(X . W) with fp32 accumulation, the values nl_gemm would store.
 *
 * nl_lce_fwd: loss[m] = lse[m] - l[m, t[m]], lse[m] = logsumexp_v l[m, v]
 * (NaN loss for a target outside [0, V)). The GEMM reduces each 256-column
 * tile of logits to per-row (max, sum) partials in its epilogue; a second
 * kernel merges them. Workspace: nl_lce_ws_bytes(M, V) bytes, 16-byte aligned. */
size_t nl_lce_ws_bytes(int M, int V);
int nl_lce_fwd(void* stream, int M, int D, int V, const nl_bf16* X, int64_t ldx,
               const nl_bf16* W, int64_t ldw, const int32_t* targets,
               float* loss, float* lse, void* ws, size_t ws_bytes);

/* dlogits[m][c] = (exp(l[m, v] - lse[m]) - [v == t[m]]) * scale * (*scale_dev)
 * for vocabulary columns v = v0 + c, c < vn (scale_dev may be NULL: factor 1),
 * written as bf16 [M][ld_dlogits]; v0 % 8 == 0 and v0 + vn <= V. The logits
 * are recomputed by the GEMM (cross_entropy.py:150-152) and never stored. The
 * caller forms dX = dlogits . W[:, v0:v0+vn]^T and dW[:, v0:v0+vn] =
 * X^T . dlogits with nl_gemm (cross_entropy.py:157-158). */
int nl_lce_bwd_dlogits(void* stream, int M, int D, int V, int v0, int vn,
                       const nl_bf16* X, int64_t ldx, const nl_bf16* W, int64_t ldw,
                       const int32_t* targets, const float* lse, float scale,
                       const float* scale_dev, nl_bf16* dlogits, int64_t ld_dlogits);

/* out[0] = mean(x[0..n)) in a fixed summation order (deterministic).
 * Replaces loss.mean() (cross_entropy.py:51). */
int nl_mean_f32(void* stream, const float* x, int n, float* out);

/* x[r, c] *= *g for r < rows, c < cols (bf16, row stride ld). Reads the scalar
 * on the device and returns without touching x when *g == 1, so the usual
 * unit cotangent costs one tiny launch. Replaces g * dlogits (cross_entropy.py:65). */
int nl_scale_bf16_by_device_scalar(void* stream, nl_bf16* x, int64_t rows, int64_t cols,
                                   int64_t ld, const float* g);

/* ======================================================================== */
/* AdamW (the optimizer of the training step)                                */
/* ======================================================================== */
/*
 * One decoupled-weight-decay Adam update of a [rows][cols] fp32 tensor (p, g,
 * m, v dense with row stride cols), following optax.adamw as called at
 * nlearn/train.py:504-505:
 *   m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g^2
 *   p = p - lr * ( (m / bc1) / (sqrt(v / bc2) + eps) + wd * p )
 * with bc1 = 1 - b1^t, bc2 = 1 - b2^t for update number t (1-based).
 * b1 and b2 are doubles, as optax's are Python floats: b and 1 - b are each
 * formed in double and rounded once to fp32 (1 - 0.999 is 0.001f, where fp32
 * arithmetic on 0.999f would give 0.00099998713).
 * If p_bf16 != NULL the updated weight is also written there as bf16 (row
 * stride ld_bf16): the compute copy the next forward reads, so no separate
 * cast pass is needed (model.py:372-375 casts every parameter each step).
 */
int nl_adamw_step(void* stream, int64_t rows, int64_t cols, float* p, const float* g, float* m, float* v,
                  nl_bf16* p_bf16, int64_t ld_bf16, float lr, double b1, double b2, float eps, float wd,
                  float bc1, float bc2);

/* The same update over a whole parameter tree in ONE launch (the optax update
 * of train.py:504-505 applied to every leaf). The caller describes each leaf
 * once in a table of nl_adamw_tensor; nl_adamw_multi_prepare() (host only)
 * fills chunk0 and returns the launch size, and the table is then copied to
 * device memory and reused every step. The per-step scalars live in device
 * memory, hyper_dev = {lr, bc1, bc2}, so a captured HIP graph replays the
 * update with the values the host writes there before each replay.
 * p, g, m, v of a leaf are dense [rows][cols] fp32 and 16-byte aligned;
 * shadow (optional) is the bf16 copy with row stride ld_shadow. */
typedef struct nl_adamw_tensor {
  float* p;
  const float* g;
  float* m;
  float* v;
  nl_bf16* shadow;
  int64_t ld_shadow;
  int64_t rows, cols;
  int64_t chunk0;     /* first work chunk of this leaf (set by nl_adamw_multi_prepare) */
} nl_adamw_tensor;
int64_t nl_adamw_multi_prepare(int n_tensors, nl_adamw_tensor* tensors_host);
int nl_adamw_multi(void* stream, int n_tensors, const nl_adamw_tensor* tensors_dev, int64_t n_chunks,
                   const float* hyper_dev, double b1, double b2, float eps, float wd);

/* nl_adamw_multi with optax.clip_by_global_norm(max_norm) chained in front of
 * it (train.py:502-506: optax.chain(clip_by_global_norm(NLEARN_GRAD_CLIP),
 * adamw)): every gradient element is used as g while *gnorm_dev < max_norm,
 * else as (g / *gnorm_dev) * max_norm. *gnorm_dev is the global L2 norm over
 * all leaves, e.g. written by nl_global_norm on the same stream. */
int nl_adamw_multi_clip(void* stream, int n_tensors, const nl_adamw_tensor* tensors_dev, int64_t n_chunks,
                        const float* hyper_dev, double b1, double b2, float eps, float wd,
                        const float* gnorm_dev, float max_norm);

/* out[0] = sqrt(sum_i g[i]^2) over a dense fp32 vector (16-byte aligned; the
 * model's whole gradient buffer, whose padding is zero): optax.global_norm as
 * clip_by_global_norm uses it. Fixed summation order (bitwise reproducible);
 * workspace of nl_global_norm_ws_bytes(n) bytes. Two launches, no host sync. */
size_t nl_global_norm_ws_bytes(int64_t n);
int nl_global_norm(void* stream, int64_t n, const float* g, float* out, void* ws, size_t ws_bytes);

/* Gradient accumulation over micro-steps, as optax.MultiSteps does it
 * (train.py:319-325,507-508 wrap the optimizer in MultiSteps(every_k_schedule=
 * NLEARN_GRAD_ACCUM)), with the loss-scale division of train_step
 * (train.py:332-337, g / NLEARN_LOSS_SCALE) in front:
 *   u = g[i] / coef_dev[0];
 *   acc[i] = u                                   if coef_dev[1] == 1,
 *          = acc[i] + (u - acc[i]) / coef_dev[1]  otherwise,
 * with coef_dev[1] = (micro-step index) + 1: acc is the running mean of the
 * micro-steps' gradients. Both scalars are read on the device (a captured
 * graph replays with the values written before each replay). acc may equal g
 * (unscaling in place). n elements, 16-byte aligned. */
int nl_grad_accumulate(void* stream, int64_t n, float* acc, const float* g, const float* coef_dev);

/* ======================================================================== */
/* LayerNorm, bias gradients, embedding                                       */
/* ======================================================================== */
/*
 * LayerNorm over rows of a bf16 [rows][D] matrix (dense, D % 8 == 0, D <= 4096),
 * fp32 gamma / beta / statistics:
 *   s = x (+ residual; then s is rounded to bf16 and written to sum_out)
 *   y = bf16((s - mean) * rstd * gamma + beta),  rstd = 1 / sqrt(var(s) + eps)
 * mean and rstd ([rows] fp32) are saved for the backward. Folding the residual
 * add of the block into the next LayerNorm reads the residual stream once.
 * All pointers 16-byte aligned.
 *
 * Replaces layer_norm (model.py:228-241) and the residual adds of
 * block_forward (model.py:315-324); the benchmark layout normalises with a
 * mean-centred LayerNorm with learned beta (the current file uses RMSNorm).
 */
int nl_layernorm_fwd(void* stream, int rows, int D, const nl_bf16* x, const nl_bf16* residual,
                     nl_bf16* sum_out, const float* gamma, const float* beta, float eps,
                     nl_bf16* y, float* mean, float* rstd);

/* Backward of nl_layernorm_fwd (the autodiff of model.py:228-241):
 *   dx = rstd * (g - mean(g) - xh * mean(g * xh)) (+ dres),  g = dy * gamma,
 *   xh = (x - mean) * rstd, with x the normalised input (sum_out when fused);
 *   dgamma (+)= sum_rows dy * xh,  dbeta (+)= sum_rows dy   (accumulate != 0 adds).
 * dres (may be NULL) is the gradient arriving through the residual branch.
 * The parameter sums use a workspace of nl_layernorm_bwd_ws_bytes() bytes and
 * are reduced in a fixed order (bitwise reproducible). */
size_t nl_layernorm_bwd_ws_bytes(int rows, int D);
int nl_layernorm_bwd(void* stream, int rows, int D, const nl_bf16* dy, const nl_bf16* x,
                     const float* mean, const float* rstd, const float* gamma, const nl_bf16* dres,
                     nl_bf16* dx, float* dgamma, float* dbeta, int accumulate, void* ws, size_t ws_bytes);

/* nl_layernorm_bwd with the parameter sums deferred, for a chain of LayerNorm
 * backwards whose dgamma / dbeta only an optimizer reads later (the model's 9
 * per step): dx is formed as above, but this call's sums stay as partial rows
 * in ws (keep it until they are reduced), and the same launch reduces the
 * partials that an earlier deferred call left in prev_ws (prev_rows x prev_D;
 * prev_ws NULL: nothing to reduce) into prev_dgamma / prev_dbeta (+= if
 * prev_accumulate). One kernel launch instead of two per LayerNorm; the sums
 * are those of nl_layernorm_bwd, bit for bit. */
int nl_layernorm_bwd_deferred(void* stream, int rows, int D, const nl_bf16* dy, const nl_bf16* x,
                              const float* mean, const float* rstd, const float* gamma, const nl_bf16* dres,
                              nl_bf16* dx, void* ws, size_t ws_bytes, int prev_rows, int prev_D,
                              const void* prev_ws, float* prev_dgamma, float* prev_dbeta, int prev_accumulate);

/* Reduces the partial rows a deferred call left in ws (rows, D as in that call)
 * into dgamma / dbeta (+= if accumulate): the last link of such a chain. */
int nl_layernorm_param_sums(void* stream, int rows, int D, const void* ws, float* dgamma, float* dbeta,
                            int accumulate);

/* out[c] (+)= sum_r x[r][c] over a bf16 [rows][ld] matrix: the bias gradients
 * db = sum_rows dY of the FFN biases (autodiff of model.py:266-277 with the
 * benchmark's b1, b2). Fixed summation order; workspace nl_colsum_ws_bytes(). */
size_t nl_colsum_ws_bytes(int rows, int cols);
int nl_colsum_bf16(void* stream, int rows, int cols, const nl_bf16* x, int64_t ld, float* out,
                   int accumulate, void* ws, size_t ws_bytes);

/* out[b][s][:] = bf16(tok[ids[b][s]][:] + pos[s][:]), fp32 tables [vocab][D] and
 * [>= seq][D], D % 4 == 0; an id outside [0, vocab) gives a NaN row.
 * Replaces embed (model.py:75-85) with the benchmark's learned position table. */
int nl_embedding_fwd(void* stream, int batch, int seq, int D, int vocab, const int32_t* ids,
                     const float* tok, const float* pos, nl_bf16* out);

/* dtok[v] = sum of dx[t] over the tokens t with ids[t] == v, in increasing t
 * (deterministic, no atomics: np.add.at's order), for every row v of the
 * [vocab][D] table: rows no token uses are written as zero, so dtok needs no
 * zeroing first. dpos[s] (+)= sum_b dx[b][s] in batch order for s < seq (rows of
 * dpos at or past seq are not touched). D % 4 == 0, D <= 4096; dtok 16-byte and
 * dx 8-byte aligned. Three launches (the tokens of each vocabulary bucket
 * counted, then listed in token order, then the rows) over a workspace of
 * nl_embedding_bwd_ws_bytes() bytes, 16-byte aligned (unused with no tokens):
 * one 8-byte entry per token plus 32 bytes per vocabulary bucket (at most 256
 * buckets).
 * The autodiff of the gather in model.py:75-85. */
size_t nl_embedding_bwd_ws_bytes(int batch, int seq, int D, int vocab);
int nl_embedding_bwd(void* stream, int batch, int seq, int D, int vocab, const int32_t* ids,
                     const nl_bf16* dx, float* dtok, float* dpos, int accumulate_pos, void* ws,
                     size_t ws_bytes);

#ifdef __cplusplus
}
#endif
#endif /* NLEARN_HIP_H */
