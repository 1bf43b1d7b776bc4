/*
 * mi_gemm.h -- C ABI of the MI355X (gfx950) GEMM core.
 *
 * Drop-in boundary for the matmul operator layer of the reference C++ engine
 * (rahul238xaviers/large-language-model, cpp/).  Every entry point below states
 * the reference interface it replaces.  Plain pointers and sizes only: all
 * matrix pointers are DEVICE pointers owned by the caller; `stream` is a
 * hipStream_t (NULL = legacy default stream).  Every call is asynchronous on
 * `stream` and returns a status code (0 = MI_OK) after validating its
 * arguments on the host; nothing here allocates device memory.
 *
 * Layout conventions (row-major, as in the reference, gemm_bf16.metal:45,63):
 *   op(A)[m,k] = transA ? A[k*lda + m] : A[m*lda + k]     (op(A) is M x K)
 *   op(B)[k,n] = transB ? B[n*ldb + k] : B[k*ldb + n]     (op(B) is K x N)
 *   C[m,n] at C[m*ldc + n]
 * Engine layout (weights W[in,out], Y = X*W) is transA=0, transB=0 (NN);
 * nn.Linear layout (W[out,in], Y = X*W^T) is NT; weight gradients dW = X^T*dY
 * are TN.
 *
 * Epilogue, applied in fp32 to the fp32 accumulator acc = sum_k op(A)*op(B):
 *   t = alpha*acc                         (dual-B: t = SiLU(alpha*acc_g) * (alpha*acc_u))
 *   t *= row_scale[m]                     if epi->row_scale
 *   t += bias[n]                          if epi->bias
 *   t += beta * C[m,n]                    if beta != 0 (C read in its own dtype)
 *   t += R[m*ldr + n]                     if epi->residual
 *   C[m,n] = t   (fp32, or bf16 rounded to nearest even)
 * with SiLU(x) = x / (1 + exp(-x)).
 */
#ifndef MI_GEMM_H
#define MI_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mi_dtype { MI_F32 = 0, MI_BF16 = 1, MI_F16 = 2 /* checkpoint sources only */ } mi_dtype;

typedef enum mi_status {
  MI_OK = 0,
  MI_ERR_SHAPE = 1,       /* negative size, inconsistent K segments, bad batch description */
  MI_ERR_LD = 2,          /* leading dimension smaller than the row it must hold */
  MI_ERR_NULL = 3,        /* required pointer is NULL */
  MI_ERR_DTYPE = 4,       /* dtype combination not supported */
  MI_ERR_UNSUPPORTED = 5, /* feature combination not supported (message says which) */
  MI_ERR_WORKSPACE = 6,   /* workspace too small for the requested split */
  MI_ERR_HIP = 7,         /* HIP runtime error (message carries hipGetErrorString) */
  MI_ERR_NO_DEVICE = 8    /* no gfx950 device visible */
} mi_status;

/* Causal structure of a batched product (GQA attention forms). */
typedef enum mi_causal {
  MI_CAUSAL_NONE = 0,
  MI_CAUSAL_OUT_LOWER = 1, /* only C[m,n] with n <= m is computed; n > m gets mask_value   */
  MI_CAUSAL_A_LOWER = 2,   /* op(A)[m,k] == 0 for k > m (within a K segment): skipped     */
  MI_CAUSAL_A_UPPER = 3    /* op(A)[m,k] == 0 for k < m (within a K segment): skipped     */
} mi_causal;

/* Optional fused prologue/epilogue operands.  Any field may be NULL / 0. */
typedef struct mi_epilogue {
  const void* bias;      /* [N] row-broadcast bias, dtype bias_dtype                       */
  int32_t bias_dtype;    /* mi_dtype                                                        */
  const void* residual;  /* R[M, ldr] added after beta*C, dtype residual_dtype              */
  int32_t residual_dtype;
  int64_t ldr;
  const void* B2;        /* dual-B SiLU gate: C = SiLU(A*B) (.) (A*B2), B2 laid out as B     */
  const void* A2;        /* SiLU-gate prologue: op(A) := SiLU(A) (.) A2, A2 laid out as A    */
  const float* row_scale; /* [M] fp32 factor per output row (a folded RMSNorm: 1/rms of
                             row m, mi_rmsnorm_fwd with y = NULL); one problem, no B2       */
} mi_epilogue;

/*
 * Strided batch: problem z in [0, batch) is split as zo = z / heads,
 * zi = z % heads and operand X is offset by  zo*X_outer + (zi / X_group)*X_inner
 * elements.  X_group > 1 maps several query heads onto one shared KV head
 * (GQA: kv_h = h / (nH/nKV), Attention.cpp:241).  The reduction dimension is
 * k_segments segments of K each; segment j of A / B starts seg_a / seg_b
 * elements after segment 0 (the KV-group reduction of dK/dV, Attention.cpp:332,
 * 344-345, is one product whose K runs over the nH/nKV query heads).
 */
typedef struct mi_batch {
  int64_t batch, heads;
  int64_t a_outer, a_inner, a_group;
  int64_t b_outer, b_inner, b_group;
  int64_t c_outer, c_inner, c_group;
  int64_t r_outer, r_inner;  /* residual batch strides (group 1) */
  int64_t k_segments;        /* >= 1 */
  int64_t seg_a, seg_b;
  int32_t causal;            /* mi_causal */
  float mask_value;          /* written where MI_CAUSAL_OUT_LOWER masks */
} mi_batch;

/* Initialise the runtime on the current device; idempotent.  Returns
 * MI_ERR_NO_DEVICE when no gfx950 GPU is visible.  Replaces
 * metal_bridge::initialize / is_available (MetalBridge.hpp:20-21). */
int mi_init(void);

/* Text of the last error raised on the calling thread ("" if none). */
const char* mi_last_error(void);

/* Library version string. */
const char* mi_version(void);

/* Workspace bytes mi_gemm / mi_gemm_batched would use for split-K on this
 * problem when given unlimited workspace (0 if it would not split). */
size_t mi_gemm_workspace_size(int transA, int transB, int64_t M, int64_t N, int64_t K,
                              int32_t dtype_in, int32_t dtype_c, int64_t batch);

/*
 * General GEMM with fused epilogue.  A and B share one input dtype (MI_BF16 or
 * MI_F32); C is MI_BF16 or MI_F32.  workspace may be NULL (then no split-K).
 * With epi->A2 (SiLU-gate prologue), bf16 inputs, transA = 0 and a 16-byte
 * aligned workspace of at least M*K*2 bytes, SiLU(A) (.) A2 is written to the
 * workspace in one pass (bf16, as the prologue rounds it) and the GEMM runs on
 * it with the rest of the workspace; otherwise the prologue is applied as each
 * A tile is loaded.
 * Replaces metal_bridge::gemm_bf16 (MetalBridge.hpp:39-42), gemm_proj (:121),
 * gemm_backward (:122-123), gemm_proj_trans_b (:124-125), gemm_ffn (:119-120,
 * via epi->B2) and fused_swiglu_gemm (:44-46, via epi->A2), and the residual
 * pass residual_add (:78) when fused via epi->residual or beta = 1.
 */
int mi_gemm(void* stream, int transA, int transB, int64_t M, int64_t N, int64_t K,
            float alpha, const void* A, int64_t lda, const void* B, int64_t ldb,
            int32_t dtype_in, float beta, void* C, int64_t ldc, int32_t dtype_c,
            const mi_epilogue* epi, void* workspace, size_t workspace_bytes);

/*
 * mi_gemm for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart
 * in the reference.  Same arguments, arithmetic and kernels as mi_gemm given a
 * workspace of mi_gemm_workspace_size bytes, minus the workspace: split-K partials
 * go to a static device array of MI_NOALLOC_SCRATCH_BYTES that the library holds
 * on each GPU it runs on until the process ends (its address is set up by mi_init
 * or the first call on a device).  A split-K plan writes at most two 128x128 fp32
 * tiles of partials per CU, 32 MiB on a 256-CU MI355X, so every problem fits; a
 * plan needing more (a larger device) fails with MI_ERR_WORKSPACE.  With the
 * SiLU-gate prologue (epi->A2) it runs the plan mi_gemm makes given no workspace
 * (the activation applied while each A tile is loaded, no split): the two-pass
 * form mi_gemm takes when its workspace holds the M x K activation does not fit
 * the scratch.  Calls no allocating routine.  Every call on a
 * GPU shares that GPU's array: calls that overlap in time on one GPU (different
 * streams, or different host threads) race and must be serialised by the caller.
 * Not recorded by the profiler.
 */
#define MI_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int mi_gemm_noalloc(void* stream, int transA, int transB, int64_t M, int64_t N, int64_t K,
                    float alpha, const void* A, int64_t lda, const void* B, int64_t ldb,
                    int32_t dtype_in, float beta, void* C, int64_t ldc, int32_t dtype_c,
                    const mi_epilogue* epi);

/*
 * Strided-batched GEMM with GQA head mapping, K segments and causal skipping.
 * Replaces the per-slice gemm_bf16 loop of Tensor::matmul's batched branch
 * (Tensor.cpp:196-227) and the batched QK^T / P*V / dV / dP / dQ / dK products
 * of GQA attention (Attention.cpp:236-280, 292-348; flash_attn_fwd and
 * fused_attn_bwd, MetalBridge.hpp:49-57).
 */
int mi_gemm_batched(void* stream, int transA, int transB, int64_t M, int64_t N, int64_t K,
                    float alpha, const void* A, int64_t lda, const void* B, int64_t ldb,
                    int32_t dtype_in, float beta, void* C, int64_t ldc, int32_t dtype_c,
                    const mi_batch* batch, const mi_epilogue* epi, void* workspace,
                    size_t workspace_bytes);

/* a[i] += b[i] for i < n (dtype MI_F32 or MI_BF16).  Replaces
 * metal_bridge::residual_add (MetalBridge.hpp:78, residual_add.metal:15-28). */
int mi_residual_add(void* stream, void* a, const void* b, int64_t n, int32_t dtype);

/*
 * Row softmax of causal attention scores, in place on S [rows, T] (row r of a
 * head is query position r % T): P[q,k] = exp(S[q,k]-max)/sum over k <= q,
 * zero for k > q (Attention.cpp:261-266).  S dtype MI_F32 or MI_BF16.
 */
int mi_softmax_causal(void* stream, void* S, int64_t rows, int64_t T, int64_t ld,
                      int32_t dtype);

/*
 * Softmax backward for attention: dS = P (.) (dP - rowsum(P (.) dP)) * scale,
 * written over dP (Attention.cpp:336-345).  Same shape conventions as above.
 */
int mi_softmax_bwd(void* stream, const void* P, void* dP, int64_t rows, int64_t T,
                   int64_t ld, float scale, int32_t dtype);

/* Output layouts of mi_flash_attn_fwd. */
typedef enum mi_attn_layout {
  MI_ATTN_O_BHTD = 0, /* O[b][h][t][c]           (flash_attn_fwd.metal)            */
  MI_ATTN_O_BTHD = 1  /* O[b][t][h*d + c]        (Attention.cpp:270-278, [B,T,nH*d]) */
} mi_attn_layout;

/*
 * Fused GQA attention forward: O = softmax(Q K^T / sqrt(d), causal k <= q) V with
 * query head h reading KV head h / (n_heads / n_kv), S and P kept on chip (online
 * softmax).  Q [batch, n_heads, seq_len, d], K and V [batch, n_kv, seq_len, d], O
 * per o_layout, all bf16 and 16-byte aligned; lse (optional, fp32 [batch,
 * n_heads, seq_len]) receives each row's natural-log log-sum-exp of the scaled
 * scores, for a backward pass.  causal = 0 attends to every key.  head_dim 64
 * (the reference kernel's compiled size, flash_attn_fwd.metal:31) or 128; n_heads
 * a multiple of n_kv.  Replaces metal_bridge::flash_attn_fwd
 * (MetalBridge.hpp:49-51) and the forward of Attention::forward
 * (Attention.cpp:236-280).
 */
int mi_flash_attn_fwd(void* stream, const void* Q, const void* K, const void* V, void* O,
                      float* lse, int64_t batch, int64_t n_heads, int64_t n_kv, int64_t seq_len,
                      int64_t head_dim, int32_t causal, int32_t o_layout);

/*
 * Fused GQA attention backward (FlashAttention-2 form), causal as in the
 * forward: from Q, K, V, the forward's O and lse and the output gradient dO,
 * computes dQ [batch, n_heads, seq_len, d] and dK, dV [batch, n_kv, seq_len, d]
 * (bf16), dK/dV summed over the n_heads/n_kv query heads of each KV head.  O
 * and dO use o_layout; delta is caller workspace of batch*n_heads*seq_len fp32
 * (receives rowsum(dO * O)).  Deterministic (no atomics).  head_dim 64 or 128.
 * With workspace of mi_flash_attn_bwd_workspace_size bytes (16-byte aligned;
 * seq_len a multiple of 8, at most 32767) the dK/dV kernel also writes dS^T there and dQ is
 * one batched GEMM (5 MFMA products); with NULL / too little workspace a dQ
 * kernel recomputes S and dP instead (7 products).  Replaces
 * metal_bridge::fused_attn_bwd (MetalBridge.hpp:54-57; that kernel recomputes
 * the forward itself, this one takes the forward's O and lse) and the backward
 * of Attention::backward (Attention.cpp:292-348).
 */
int mi_flash_attn_bwd(void* stream, const void* Q, const void* K, const void* V, const void* O,
                      const void* dO, const float* lse, void* dQ, void* dK, void* dV, float* delta,
                      int64_t batch, int64_t n_heads, int64_t n_kv, int64_t seq_len,
                      int64_t head_dim, int32_t causal, int32_t o_layout, void* workspace,
                      size_t workspace_bytes);

/* Workspace bytes for the dS^T form of mi_flash_attn_bwd: batch*n_heads*seq_len^2
 * bf16 for dS^T, then batch*n_heads*seq_len*128 fp32 (enough for head_dim 128) for the partial dK / dV sums
 * of the balanced dK/dV schedule (a workspace holding dS^T only runs the dS^T form
 * with one workgroup per key block); 0 when the form does not apply (seq_len not a
 * multiple of 8, or above 32767). */
size_t mi_flash_attn_bwd_workspace_size(int64_t batch, int64_t n_heads, int64_t seq_len);

/*
 * mi_flash_attn_fwd / mi_flash_attn_bwd with the softmax scale given (the two
 * functions above use 1/sqrt(head_dim), Attention.cpp:208).  For a head dimension
 * d that is neither 64 nor 128 (a multiple of 8 below 128), copy Q, K, V (and dO)
 * into rows of the next kernel size (64 or 128 columns) whose columns past d are
 * zero and pass scale = 1/sqrt(d): the zero columns add exact zeros to every
 * score, and the output and gradient columns past d come out zero.  The C++
 * bridge does this for flash_attn_fwd / fused_attn_bwd.  scale must be positive
 * and finite.
 */
int mi_flash_attn_fwd_scaled(void* stream, const void* Q, const void* K, const void* V, void* O,
                             float* lse, int64_t batch, int64_t n_heads, int64_t n_kv, int64_t seq_len,
                             int64_t head_dim, int32_t causal, int32_t o_layout, float scale);
int mi_flash_attn_bwd_scaled(void* stream, const void* Q, const void* K, const void* V, const void* O,
                             const void* dO, const float* lse, void* dQ, void* dK, void* dV, float* delta,
                             int64_t batch, int64_t n_heads, int64_t n_kv, int64_t seq_len,
                             int64_t head_dim, int32_t causal, int32_t o_layout, void* workspace,
                             size_t workspace_bytes, float scale);

/*
 * Softmax cross-entropy over rows of logits, the loss after the LM head.  For
 * row r (a token) with target y = targets[r]:
 *   p[v] = exp(x[v] - max x) / sum_v exp(x[v] - max x)
 *   row_loss[r] = -log(max(p[y], 1e-15))
 *   grad[r, v]  = scale * (p[v] - [v == y])           (if grad is not NULL)
 *   *loss_out   = scale * sum_r row_loss[r]            (if loss_out is not NULL)
 * logits [rows, ld_logits] and grad [rows, ld_grad] are MI_BF16 or MI_F32 (fp32
 * arithmetic either way); grad may be the logits array itself (same dtype and
 * leading dimension: the gradient overwrites the logits) but must not
 * otherwise overlap it.  targets, row_loss [rows] and loss_out [1] are device
 * memory; row_loss is required.  The reference's scale is 1 / rows.  A target
 * outside [0, vocab) gives a NaN row loss.  Deterministic (fixed-order
 * reductions, no atomics); rows == 0 or vocab == 0 is a no-op.  Replaces
 * metal_bridge::cross_entropy (MetalBridge.hpp:89-91, cross_entropy.metal) and
 * CrossEntropyLoss::forward / backward (Loss.hpp, Loss.cpp:43-195).
 */
int mi_cross_entropy(void* stream, const void* logits, int32_t logits_dtype, int64_t ld_logits,
                     const uint32_t* targets, int64_t rows, int64_t vocab, float scale,
                     float* row_loss, float* loss_out, void* grad, int32_t grad_dtype,
                     int64_t ld_grad);

/*
 * LM head + softmax cross-entropy without the [rows, vocab] logits: the logits
 * are made one vocabulary chunk of `chunk` columns at a time into the
 * workspace, and never exist whole.  X [rows, ldx] is the final hidden state and
 * W the output projection, both MI_BF16: w_layout 0 is W [hidden, ldw] (the
 * reference's output_projection_, logits = X W), w_layout 1 is W [vocab, ldw]
 * (a tied embedding table, logits = X W^T).  Per row r with y = targets[r] the
 * results are those of mi_cross_entropy on the bf16 logits (same definitions
 * of row_loss, loss_out, scale and a target outside [0, vocab)), and then
 *   dX = G W^T (layout 0) or G W (layout 1)              (if dX is not NULL)
 *   dW = dw_beta dW + X^T G (layout 0) or G^T X (layout 1) (if dW is not NULL)
 * with G = scale * (softmax - onehot) rounded to bf16.  Pass 1 runs the logits
 * GEMM of each chunk and merges its (max, sum exp) into per-row running values;
 * pass 2, when dX or dW is requested, visits the chunks last first, recomputes
 * each chunk's logits (the last chunk's are still in the workspace), overwrites
 * them with G and runs the dX and dW GEMMs of the chunk (dX accumulated in
 * fp32, in the workspace when dX is MI_BF16).  dX is MI_BF16 or MI_F32
 * [rows, lddx]; dW is MI_BF16 or MI_F32 with W's shape.  chunk <= 0 or >= vocab
 * means one chunk (no recomputation).  workspace (device memory, not overlapping
 * any argument) holds at least mi_lm_head_xent_workspace_size bytes; bytes
 * beyond that are split-K workspace for the GEMMs.  Deterministic.  Replaces the
 * output projection and loss of the reference's step: final_h.matmul(
 * output_projection_) (Transformer.cpp:193-194), CrossEntropyLoss::forward /
 * backward (Loss.cpp:43-195), accumulate_output_projection_grads and
 * gemm_proj_trans_b for grad_final_h (Transformer.cpp:600-616).
 */
size_t mi_lm_head_xent_workspace_size(int64_t rows, int64_t hidden, int64_t vocab, int64_t chunk,
                                      int32_t dx_dtype);
int mi_lm_head_xent(void* stream, const void* X, int64_t ldx, const void* W, int32_t w_layout, int64_t ldw,
                    const uint32_t* targets, int64_t rows, int64_t hidden, int64_t vocab, float scale,
                    float* row_loss, float* loss_out, void* dX, int32_t dx_dtype, int64_t lddx, void* dW,
                    int32_t dw_dtype, int64_t lddw, float dw_beta, int64_t chunk, void* workspace,
                    size_t workspace_bytes);

/*
 * RMSNorm forward over rows of dims values: with residual != NULL, first
 * x += residual (x updated in place, in its own dtype), then
 *   y = x / sqrt(sum(x^2)/dims + eps) * weight
 * computed in fp32.  x, residual, y are [rows, ld] of `dtype` (MI_BF16 or
 * MI_F32), weight [dims] of w_dtype; rstd (optional, fp32 [rows]) receives
 * 1/rms per row.  y may be x itself; arrays must otherwise not overlap.  y = NULL
 * (rstd required) computes only x += residual and rstd: the norm is then folded
 * into the next GEMM, rmsnorm(x) W = diag(rstd) x W' with W' = diag(weight) W
 * (mi_rmsnorm_fold_weight), rstd passed as that GEMM's epi->row_scale.
 * Replaces metal_bridge::rms_norm_forward (MetalBridge.hpp:60-61,
 * rms_norm_forward.metal; RMSNorm::forward, RMSNorm.cpp:48-75) and
 * metal_bridge::fused_add_norm (MetalBridge.hpp:79-81, fused_add_norm.metal;
 * h += out; ffn_in = rmsnorm(h), Transformer.cpp:150-158).
 */
int mi_rmsnorm_fwd(void* stream, void* x, const void* residual, const void* weight, int32_t w_dtype,
                   void* y, float* rstd, int64_t rows, int64_t dims, int64_t ld, int32_t dtype,
                   float eps);

/* Workspace bytes mi_rmsnorm_bwd needs when it computes dw. */
size_t mi_rmsnorm_bwd_workspace_size(int64_t rows, int64_t dims);

/*
 * W_out[k, n] = weight[k] * W[k, n] for k < K, n < N (fp32 product stored in W's
 * dtype, bf16 rounded to nearest even): the RMSNorm weight moved into the rows of
 * the GEMM that consumes the norm (the QKV and gate/up projections,
 * Transformer.cpp:147-162, Attention.cpp:196-201), so that
 *   rmsnorm(x) W = diag(1/rms) x W_out.
 * With mi_rmsnorm_fwd's statistic-only mode and the GEMM's epi->row_scale this
 * replaces the pair fused_add_norm / rms_norm_forward -> matmul
 * (MetalBridge.hpp:60-61,79-81 then Tensor::matmul) by a row statistic and one
 * GEMM on x itself: the normalised activations are never written.  W_out may be W
 * (ld_out == ldw) or disjoint from it.  dtype MI_BF16 or MI_F32; weight MI_BF16
 * or MI_F32.
 */
int mi_rmsnorm_fold_weight(void* stream, const void* weight, int32_t w_dtype, const void* W, int64_t ldw,
                           int64_t K, int64_t N, int32_t dtype, void* W_out, int64_t ld_out);

/*
 * RMSNorm backward: with xhat = x / rms and rms = sqrt(sum(x^2)/dims + eps),
 *   dx = (dy*w - xhat * mean(dy*w*xhat)) / rms  [+ residual_grad]
 *   dw = dw_beta * dw + sum over rows of dy * xhat     (if dw is not NULL)
 * dy, x, residual_grad, dx are [rows, ld] of `dtype`; weight [dims] of
 * w_dtype; dw [dims] of dw_dtype.  dx may be dy, x or residual_grad itself.
 * dw needs workspace of mi_rmsnorm_bwd_workspace_size bytes; it is summed in
 * a fixed order (bit-identical across launches).  Replaces
 * metal_bridge::rms_norm_backward (MetalBridge.hpp:62-64, rms_norm_backward.metal;
 * RMSNorm::backward, RMSNorm.cpp:77-180) and metal_bridge::fused_backward_add_norm
 * (MetalBridge.hpp:82-85, fused_backward_add_norm.metal, Transformer.cpp:441-466).
 */
int mi_rmsnorm_bwd(void* stream, const void* dy, const void* x, const void* weight, int32_t w_dtype,
                   const void* residual_grad, void* dx, void* dw, int32_t dw_dtype, float dw_beta,
                   int64_t rows, int64_t dims, int64_t ld, int32_t dtype, float eps,
                   void* workspace, size_t workspace_bytes);

/*
 * Weight conversion for checkpoint loading: rows [row0, row0 + rows) x columns
 * [0, cols) of a row-major source matrix (leading dimension src_ld, dtype MI_F32,
 * MI_BF16 or MI_F16) into dst (MI_F32, or MI_BF16 rounded to nearest even):
 *   dst[r*dst_ld + c] = src[(row0 + r)*src_ld + c]      transpose == 0
 *   dst[c*dst_ld + r] = src[(row0 + r)*src_ld + c]      transpose != 0
 * Both pointers are device memory and must not overlap.  One launch covers the
 * slice + transpose + widening the reference loader does on the CPU for a
 * Python/MLX checkpoint: [out, in] -> [in, out] and the row ranges of the fused
 * wqkv / w12 matrices (Checkpoint.cpp:28-75 bf16_to_f32 / f16_to_f32, :77-83
 * transpose_matrix, :407-530 load_python_tensor / load_python_fused_tensor).
 */
int mi_convert_matrix(void* stream, const void* src, int32_t src_dtype, int64_t src_ld, int64_t row0,
                      int64_t rows, int64_t cols, int32_t transpose, void* dst, int32_t dst_dtype,
                      int64_t dst_ld);

/* One conversion of mi_convert_matrices: the arguments of mi_convert_matrix. */
typedef struct mi_convert_job {
  const void* src;
  int32_t src_dtype, transpose;
  int64_t src_ld, row0, rows, cols;
  void* dst;
  int32_t dst_dtype, reserved; /* reserved: 0 */
  int64_t dst_ld;
} mi_convert_job;

/*
 * n conversions as mi_convert_matrix would do them one by one, in as few launches
 * as the dtype pairs allow (one launch per (src_dtype, dst_dtype) pair and 16
 * jobs).  Replaces the conversions of load_python_fused_tensor and
 * load_python_tensor (Checkpoint.cpp:407-530): the loaders here make one call per
 * file tensor, so the three row ranges of a fused wqkv (or the two of a w12) go
 * out in one launch; a caller with several matrices already on the device can
 * pass them all in one call.  Every job is checked first (nothing runs if one
 * fails, and the message names the job; the reserved field must be 0); sources
 * may share bytes (row ranges of one fused matrix), but no destination may
 * overlap another job's source or destination, since the tiles of a launch run
 * in any order.
 */
int mi_convert_matrices(void* stream, const mi_convert_job* jobs, int64_t n);

/*
 * Describe the kernel mi_gemm_batched would launch for this problem (tile,
 * loader, split-K factor) as text into buf (always NUL-terminated), for packed
 * operands (leading dimension = contiguous extent) at 16-byte-aligned addresses.
 * For measurement and logging; no reference counterpart.  epi_mode: 0 plain,
 * 1 dual-B, 2 SiLU-gate prologue.
 */
int mi_gemm_describe(int transA, int transB, int64_t M, int64_t N, int64_t K, int32_t dtype_in,
                     int64_t batch, int32_t epi_mode, size_t workspace_bytes, char* buf,
                     size_t buf_len);

/* Synchronise `stream`; replaces metal_bridge::end_scope's wait
 * (MetalBridge.hpp:29-30, MetalBridge.mm:2176-2225). */
int mi_stream_sync(void* stream);

/*
 * Per-call GEMM profiler.  Replaces GemmProfiler (gemm_profiler.hpp:18-117, fed
 * by MetalBridge.mm:1408-1411) and the bridge counters accum_gpu_time_ms /
 * count_gpu_calls / reset_profile_stats (MetalBridge.hpp:141-145).  While
 * enabled, every mi_gemm / mi_gemm_batched call records its problem, the plan
 * it ran and the GPU time between two HIP events placed on its stream around
 * its launches (the reference timed host-side encoding).  Off by default: the
 * events cost a few microseconds per call.
 */
typedef struct mi_gemm_record {
  int64_t M, N, K, batch;
  int32_t transA, transB, dtype_in, dtype_c;
  int32_t splits;       /* split-K factor of the plan (1 = none)                 */
  double gpu_ms;        /* GPU time of the call's kernels                          */
  char kernel[64];      /* the plan, in mi_gemm_describe's words                   */
} mi_gemm_record;

/* Turn recording on (on != 0) or off; returns the previous state. */
int mi_profiler_enable(int on);
/* GemmProfiler::begin_step: drop the records kept so far (their times stay in
 * the totals). */
int mi_profiler_begin_step(void);
/* Number of records since the last begin_step. */
int64_t mi_profiler_count(void);
/* Record i (0-based, call order); waits for that call's kernels to finish. */
int mi_profiler_record(int64_t i, mi_gemm_record* out);
/* accum_gpu_time_ms / count_gpu_calls: GPU time and number of recorded calls
 * since the last reset (waits for pending records). */
int mi_profiler_totals(double* gpu_ms, int64_t* calls);
/* reset_profile_stats: restart the totals from zero (records are kept). */
int mi_profiler_reset(void);

#ifdef __cplusplus
}
#endif
#endif /* MI_GEMM_H */
