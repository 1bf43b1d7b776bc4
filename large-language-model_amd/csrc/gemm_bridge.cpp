// gemm_bridge.cpp -- C++ mirror of the reference GEMM operator layer over the
// C ABI (declarations and the reference citations are in include/gemm_bridge.hpp).
#include "../../include/gemm_bridge.hpp"
#include "mi_convert.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>

namespace mi_bridge {
namespace {

thread_local int t_status = MI_OK;
thread_local bool t_in_scope = false;
thread_local hipStream_t t_stream = nullptr;
// Split-K workspace owned by the bridge, grown to the largest size a call asked
// for; the library itself never allocates.
thread_local void* t_ws = nullptr;
thread_local size_t t_ws_bytes = 0;

void* grow_workspace(size_t need, size_t* bytes) {
  if (need > t_ws_bytes) {
    if (t_ws) {
      // the stream may still use the old buffer
      if (hipStreamSynchronize(t_stream) != hipSuccess) return *bytes = 0, nullptr;
      (void)hipFree(t_ws);
    }
    t_ws = nullptr;
    t_ws_bytes = 0;
    if (hipMalloc(&t_ws, need) != hipSuccess) return *bytes = 0, nullptr;
    t_ws_bytes = need;
  }
  *bytes = t_ws_bytes;
  return t_ws;
}

void* workspace_for(int ta, int tb, size_t M, size_t N, size_t K, int dt_in, int dt_c,
                    size_t* bytes) {
  return grow_workspace(
      mi_gemm_workspace_size(ta, tb, (int64_t)M, (int64_t)N, (int64_t)K, dt_in, dt_c, 1), bytes);
}

// Attention state for fused_attn_bwd (O, log-sum-exp, D), grown like the split-K
// workspace; bytes = O bytes, floats = rows.
thread_local void* t_att_o = nullptr;
thread_local float* t_att_f = nullptr;
thread_local size_t t_att_rows = 0, t_att_o_bytes = 0;

hipStream_t get_stream();

bool attention_state(size_t o_bytes, size_t rows) {
  if (o_bytes <= t_att_o_bytes && rows <= t_att_rows) return true;
  if (t_att_o || t_att_f) {
    if (hipStreamSynchronize(get_stream()) != hipSuccess) return false;
    (void)hipFree(t_att_o);
    (void)hipFree(t_att_f);
  }
  t_att_o = nullptr;
  t_att_f = nullptr;
  t_att_o_bytes = t_att_rows = 0;
  if (hipMalloc(&t_att_o, o_bytes) != hipSuccess) return false;
  if (hipMalloc((void**)&t_att_f, 2 * rows * sizeof(float)) != hipSuccess) return false;
  t_att_o_bytes = o_bytes;
  t_att_rows = rows;
  return true;
}

// cross_entropy state: per-row losses and the loss scalar on the device, and the
// host copies a scope still owes its callers (the reference's copy-back tasks,
// MetalBridge.mm:1846-1900: loss_out is written once the work has run).
thread_local float* t_ce_dev = nullptr;  // [rows + 1]: row losses, then the loss
thread_local size_t t_ce_rows = 0;
thread_local float* t_ce_host = nullptr;  // pinned staging, CE_PENDING entries
constexpr int CE_PENDING = 64;
thread_local float* t_ce_dst[CE_PENDING];
thread_local int t_ce_n = 0;

bool ce_state(size_t rows) {
  if (!t_ce_host && hipHostMalloc((void**)&t_ce_host, CE_PENDING * sizeof(float)) != hipSuccess) {
    t_ce_host = nullptr;
    return false;
  }
  if (rows <= t_ce_rows) return true;
  if (t_ce_dev) {
    if (hipStreamSynchronize(get_stream()) != hipSuccess) return false;
    (void)hipFree(t_ce_dev);
  }
  t_ce_dev = nullptr;
  t_ce_rows = 0;
  if (hipMalloc((void**)&t_ce_dev, (rows + 1) * sizeof(float)) != hipSuccess) return false;
  t_ce_rows = rows;
  return true;
}

// Write the staged losses to their callers (after the stream has drained).
void ce_flush() {
  for (int i = 0; i < t_ce_n; ++i) *t_ce_dst[i] = t_ce_host[i];
  t_ce_n = 0;
}

hipStream_t get_stream() {
  if (!t_stream) {
    if (hipStreamCreateWithFlags(&t_stream, hipStreamNonBlocking) != hipSuccess) t_stream = nullptr;
  }
  return t_stream;
}

// Record the status; print like the reference bridge; wait when outside a scope.
void finish(const char* fn, int st) {
  t_status = st;
  if (st != MI_OK) {
    std::fprintf(stderr, "[mi_bridge] %s: %s\n", fn, mi_last_error());
    return;
  }
  if (!t_in_scope) {
    st = mi_stream_sync(get_stream());
    t_status = st;
    if (st != MI_OK) std::fprintf(stderr, "[mi_bridge] %s: %s\n", fn, mi_last_error());
  }
}

int gemm(int ta, int tb, size_t M, size_t N, size_t K, float alpha, const void* A, const void* B,
         int dt_in, float beta, void* C, int dt_c, const mi_epilogue* epi) {
  const int64_t lda = ta ? (int64_t)M : (int64_t)K;
  const int64_t ldb = tb ? (int64_t)K : (int64_t)N;
  hipStream_t st = get_stream();
  size_t ws_bytes = 0;
  void* ws = nullptr;
  if (!epi) {
    ws = workspace_for(ta, tb, M, N, K, dt_in, dt_c, &ws_bytes);
  } else if (epi->A2 && dt_in == MI_BF16) {
    // room for SiLU(A) * A2 (bf16, 256-byte rounded), which mi_gemm then writes in
    // one pass before a plain GEMM, and the split-K need of that GEMM after it
    const size_t act = (M * K * 2 + 255) / 256 * 256;
    ws = grow_workspace(act + mi_gemm_workspace_size(ta, tb, (int64_t)M, (int64_t)N, (int64_t)K, dt_in,
                                                     dt_c, 1),
                        &ws_bytes);
  }
  return mi_gemm(st, ta, tb, (int64_t)M, (int64_t)N, (int64_t)K, alpha, A, lda, B, ldb, dt_in, beta,
                 C, (int64_t)N, dt_c, epi, ws, ws_bytes);
}

}  // namespace

void initialize() { t_status = mi_init(); }
bool is_available() { return mi_init() == MI_OK; }

void begin_scope() {
  get_stream();
  t_in_scope = true;
}

void end_scope() {
  t_in_scope = false;
  t_status = mi_stream_sync(get_stream());
  if (t_status != MI_OK) std::fprintf(stderr, "[mi_bridge] end_scope: %s\n", mi_last_error());
  else ce_flush();
}

void* stream() { return (void*)get_stream(); }
int last_status() { return t_status; }

void gemm_bf16(const void* A, const void* B, void* C, size_t M, size_t N, size_t K, bool transA,
               bool transB, bool is_forward) {
  (void)is_forward;
  if (M == 0 || N == 0 || K == 0) {  // silent no-op, as MetalBridge.mm:622-623,693
    t_status = MI_OK;
    return;
  }
  finish("gemm_bf16", gemm(transA, transB, M, N, K, 1.0f, A, B, MI_BF16, 0.0f, C, MI_BF16, nullptr));
}

void fused_swiglu_gemm(const void* gate_proj, const void* up_proj, const void* B, void* C, size_t M,
                       size_t N, size_t K) {
  if (M == 0 || N == 0 || K == 0) {
    t_status = MI_OK;
    return;
  }
  mi_epilogue e;
  std::memset(&e, 0, sizeof(e));
  e.A2 = up_proj;
  finish("fused_swiglu_gemm",
         gemm(0, 0, M, N, K, 1.0f, gate_proj, B, MI_BF16, 0.0f, C, MI_BF16, &e));
}

void gemm_ffn(const float* a, const float* b_gate, const float* b_up, float* c, size_t M, size_t N,
              size_t K) {
  if (M == 0 || N == 0 || K == 0) {
    t_status = MI_OK;
    return;
  }
  mi_epilogue e;
  std::memset(&e, 0, sizeof(e));
  e.B2 = b_up;
  finish("gemm_ffn", gemm(0, 0, M, N, K, 1.0f, a, b_gate, MI_F32, 0.0f, c, MI_F32, &e));
}

void gemm_proj(const float* a, const float* b, float* c, size_t M, size_t N, size_t K) {
  if (M == 0 || N == 0 || K == 0) {
    t_status = MI_OK;
    return;
  }
  finish("gemm_proj", gemm(0, 0, M, N, K, 1.0f, a, b, MI_F32, 0.0f, c, MI_F32, nullptr));
}

void gemm_backward(const float* a_transposed, const float* b, float* c, size_t M, size_t N,
                   size_t K) {
  if (M == 0 || N == 0 || K == 0) {
    t_status = MI_OK;
    return;
  }
  finish("gemm_backward",
         gemm(1, 0, M, N, K, 1.0f, a_transposed, b, MI_BF16, 0.0f, c, MI_BF16, nullptr));
}

void gemm_backward_accumulate(const void* a_transposed, const void* b, float* c, size_t M, size_t N,
                              size_t K) {
  if (M == 0 || N == 0 || K == 0) {
    t_status = MI_OK;
    return;
  }
  finish("gemm_backward_accumulate",
         gemm(1, 0, M, N, K, 1.0f, a_transposed, b, MI_BF16, 1.0f, c, MI_F32, nullptr));
}

void gemm_proj_trans_b(const float* a, const float* b_transposed, float* c, size_t M, size_t N,
                       size_t K) {
  if (M == 0 || N == 0 || K == 0) {
    t_status = MI_OK;
    return;
  }
  finish("gemm_proj_trans_b",
         gemm(0, 1, M, N, K, 1.0f, a, b_transposed, MI_BF16, 0.0f, c, MI_BF16, nullptr));
}

namespace {

// Head dimensions above 128, or not a multiple of 8, run the materialised form
// (those below 128 run the fused kernels on padded rows, further down): S and P [B, nH, T, T]
// (and dP in the backward) in bridge-owned bf16 buffers, batched GEMMs with the
// KV-head map and causal skipping, and the row softmax kernels (Attention.cpp:236-348).
thread_local void* t_sp = nullptr;
thread_local size_t t_sp_bytes = 0;

bool sp_state(size_t bytes) {
  if (bytes <= t_sp_bytes) return true;
  if (t_sp) {
    if (hipStreamSynchronize(get_stream()) != hipSuccess) return false;
    (void)hipFree(t_sp);
  }
  t_sp = nullptr;
  t_sp_bytes = 0;
  if (hipMalloc(&t_sp, bytes) != hipSuccess) return false;
  t_sp_bytes = bytes;
  return true;
}

mi_batch attn_batch(int64_t batch, int64_t heads, int64_t ao, int64_t ai, int64_t ag, int64_t bo,
                    int64_t bi, int64_t bg, int64_t co, int64_t ci, int32_t causal, float mask) {
  mi_batch b;
  std::memset(&b, 0, sizeof(b));
  b.batch = batch; b.heads = heads;
  b.a_outer = ao; b.a_inner = ai; b.a_group = ag;
  b.b_outer = bo; b.b_inner = bi; b.b_group = bg;
  b.c_outer = co; b.c_inner = ci; b.c_group = 1;
  b.k_segments = 1;
  b.causal = causal;
  b.mask_value = mask;
  return b;
}

// P = softmax(Q K^T / sqrt(d)), causal, into P [B, nH, T, T]; O (BHTD) = P V when O is set.
int materialised_fwd(const void* Q, const void* K, const void* V, void* O, void* P, int64_t B,
                     int64_t nH, int64_t nKV, int64_t T, int64_t d) {
  const int64_t g = nH / nKV;
  hipStream_t st = get_stream();
  mi_batch bs = attn_batch(B * nH, nH, nH * T * d, T * d, 1, nKV * T * d, T * d, g, nH * T * T, T * T,
                           MI_CAUSAL_OUT_LOWER, -INFINITY);
  int s = mi_gemm_batched(st, 0, 1, T, T, d, (float)(1.0 / std::sqrt((double)d)), Q, d, K, d, MI_BF16,
                          0.0f, P, T, MI_BF16, &bs, nullptr, nullptr, 0);
  if (s == MI_OK) s = mi_softmax_causal(st, P, B * nH * T, T, T, MI_BF16);
  if (s == MI_OK && O) {
    mi_batch bo = attn_batch(B * nH, nH, nH * T * T, T * T, 1, nKV * T * d, T * d, g, nH * T * d, T * d,
                             MI_CAUSAL_A_LOWER, 0.0f);
    s = mi_gemm_batched(st, 0, 0, T, d, T, 1.0f, P, T, V, d, MI_BF16, 0.0f, O, d, MI_BF16, &bo,
                        nullptr, nullptr, 0);
  }
  return s;
}

int materialised_bwd(const void* Q, const void* K, const void* V, const void* dO, void* dQ, void* dK,
                     void* dV, int64_t B, int64_t nH, int64_t nKV, int64_t T, int64_t d) {
  const int64_t g = nH / nKV;
  const size_t sp = (size_t)(B * nH * T * T) * 2;
  if (!sp_state(2 * sp)) return MI_ERR_HIP;
  void* P = t_sp;
  void* dP = (char*)t_sp + sp;
  hipStream_t st = get_stream();
  int s = materialised_fwd(Q, K, V, nullptr, P, B, nH, nKV, T, d);
  // dV[b,kv] = sum over the group's heads of P^T dO   (TN, K = g segments of T)
  mi_batch b1 = attn_batch(B * nKV, nKV, nH * T * T, g * T * T, 1, nH * T * d, g * T * d, 1, nKV * T * d,
                           T * d, MI_CAUSAL_A_UPPER, 0.0f);
  b1.k_segments = g; b1.seg_a = T * T; b1.seg_b = T * d;
  if (s == MI_OK)
    s = mi_gemm_batched(st, 1, 0, T, d, T, 1.0f, P, T, dO, d, MI_BF16, 0.0f, dV, d, MI_BF16, &b1,
                        nullptr, nullptr, 0);
  // dP = dO V^T   (NT, KV map, causal output)
  mi_batch b2 = attn_batch(B * nH, nH, nH * T * d, T * d, 1, nKV * T * d, T * d, g, nH * T * T, T * T,
                           MI_CAUSAL_OUT_LOWER, 0.0f);
  if (s == MI_OK)
    s = mi_gemm_batched(st, 0, 1, T, T, d, 1.0f, dO, d, V, d, MI_BF16, 0.0f, dP, T, MI_BF16, &b2,
                        nullptr, nullptr, 0);
  // dS = P (dP - rowsum(P dP)) / sqrt(d), over dP
  if (s == MI_OK)
    s = mi_softmax_bwd(st, P, dP, B * nH * T, T, T, (float)(1.0 / std::sqrt((double)d)), MI_BF16);
  // dQ = dS K   (NN, KV map, causal K skipping)
  mi_batch b3 = attn_batch(B * nH, nH, nH * T * T, T * T, 1, nKV * T * d, T * d, g, nH * T * d, T * d,
                           MI_CAUSAL_A_LOWER, 0.0f);
  if (s == MI_OK)
    s = mi_gemm_batched(st, 0, 0, T, d, T, 1.0f, dP, T, K, d, MI_BF16, 0.0f, dQ, d, MI_BF16, &b3,
                        nullptr, nullptr, 0);
  // dK[b,kv] = sum over the group's heads of dS^T Q   (TN, K = g segments of T)
  mi_batch b4 = attn_batch(B * nKV, nKV, nH * T * T, g * T * T, 1, nH * T * d, g * T * d, 1, nKV * T * d,
                           T * d, MI_CAUSAL_A_UPPER, 0.0f);
  b4.k_segments = g; b4.seg_a = T * T; b4.seg_b = T * d;
  if (s == MI_OK)
    s = mi_gemm_batched(st, 1, 0, T, d, T, 1.0f, dP, T, Q, d, MI_BF16, 0.0f, dK, d, MI_BF16, &b4,
                        nullptr, nullptr, 0);
  return s;
}

// The fused kernels are built for head_dim 64 (the reference kernels' compiled size)
// and 128.  Other head dimensions that are multiples of 8 and below 128 run the next
// larger kernel on copies of the operands whose extra columns are zero, with the
// softmax scale of the real head dimension (mi_flash_attn_*_scaled): the zero columns
// add exact zeros to every score, and the extra output and gradient columns are
// discarded.  The pool holds Q, K, V, dO, O, dQ, dK, dV in rows of kd columns; every
// call writes all kd columns of its inputs (zeros past head_dim), so nothing a previous
// call left in the pool (other shapes, NaN from non-finite inputs) reaches the scores.
size_t fused_dim(size_t head_dim) {
  if (head_dim == 0 || head_dim % 8 || head_dim > 128) return 0;
  return head_dim <= 64 ? 64 : 128;
}

thread_local void* t_pad = nullptr;
thread_local size_t t_pad_bytes = 0;

bool pad_state(size_t bytes) {
  if (bytes > t_pad_bytes) {
    if (t_pad) {
      if (hipStreamSynchronize(get_stream()) != hipSuccess) return false;
      (void)hipFree(t_pad);
    }
    t_pad = nullptr;
    t_pad_bytes = 0;
    if (hipMalloc(&t_pad, bytes) != hipSuccess) return false;
    t_pad_bytes = bytes;
  }
  return true;
}

struct Padded {
  char *q, *k, *v, *o, *dout, *dq, *dk, *dv;
};

// Carve the pool for rows_q query rows and rows_kv key rows of kd bf16 each.
bool padded_buffers(size_t rows_q, size_t rows_kv, size_t kd, bool backward, Padded* b) {
  const size_t rq = (rows_q * kd * 2 + 255) / 256 * 256, rk = (rows_kv * kd * 2 + 255) / 256 * 256;
  if (!pad_state(backward ? 4 * rq + 4 * rk : 2 * rq + 2 * rk)) return false;
  char* w = (char*)t_pad;
  b->q = w; w += rq;
  b->o = w; w += rq;
  b->k = w; w += rk;
  b->v = w; w += rk;
  if (backward) {
    b->dout = w; w += rq;
    b->dq = w; w += rq;
    b->dk = w; w += rk;
    b->dv = w;
  }
  return true;
}

// rows x d bf16 -> rows x kd bf16 (zeros past d), and back (the first d columns).
int widen(const void* src, void* dst, size_t rows, size_t d, size_t kd) {
  int dev = 0;
  int cus = 0;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const hipError_t e = mig::launch_pad_rows(src, (int64_t)d, (int64_t)rows, (int64_t)d, dst, (int64_t)kd, cus,
                                            get_stream());
  if (e != hipSuccess) {
    std::fprintf(stderr, "[mi_bridge] padded attention operand: %s\n", hipGetErrorString(e));
    return MI_ERR_HIP;
  }
  return MI_OK;
}
int narrow(const void* src, void* dst, size_t rows, size_t d, size_t kd) {
  return mi_convert_matrix(get_stream(), src, MI_BF16, (int64_t)kd, 0, (int64_t)rows, (int64_t)d, 0, dst,
                           MI_BF16, (int64_t)d);
}

}  // namespace

void flash_attn_fwd(const void* Q, const void* K, const void* V, void* O, size_t batch,
                    size_t n_heads, size_t n_kv, size_t seq_len, size_t head_dim) {
  const size_t kd = fused_dim(head_dim);
  if (kd && kd != head_dim && batch && n_heads && seq_len) {
    if (n_kv == 0 || n_heads % n_kv) {
      finish("flash_attn_fwd", MI_ERR_SHAPE);
      return;
    }
    const size_t rq = batch * n_heads * seq_len, rk = batch * n_kv * seq_len;
    Padded b;
    if (!padded_buffers(rq, rk, kd, false, &b)) {
      t_status = MI_ERR_HIP;
      std::fprintf(stderr, "[mi_bridge] flash_attn_fwd: could not allocate the padded operands\n");
      return;
    }
    int st = widen(Q, b.q, rq, head_dim, kd);
    if (st == MI_OK) st = widen(K, b.k, rk, head_dim, kd);
    if (st == MI_OK) st = widen(V, b.v, rk, head_dim, kd);
    if (st == MI_OK)
      st = mi_flash_attn_fwd_scaled(get_stream(), b.q, b.k, b.v, b.o, nullptr, (int64_t)batch,
                                    (int64_t)n_heads, (int64_t)n_kv, (int64_t)seq_len, (int64_t)kd, 1,
                                    MI_ATTN_O_BHTD, (float)(1.0 / std::sqrt((double)head_dim)));
    if (st == MI_OK) st = narrow(b.o, O, rq, head_dim, kd);
    finish("flash_attn_fwd", st);
    return;
  }
  if (!kd && batch && n_heads && seq_len && head_dim) {
    if (n_kv == 0 || n_heads % n_kv) {
      finish("flash_attn_fwd", MI_ERR_SHAPE);
      return;
    }
    const size_t sp = batch * n_heads * seq_len * seq_len * 2;
    if (!sp_state(sp)) {
      t_status = MI_ERR_HIP;
      std::fprintf(stderr, "[mi_bridge] flash_attn_fwd: could not allocate S/P\n");
      return;
    }
    finish("flash_attn_fwd", materialised_fwd(Q, K, V, O, t_sp, (int64_t)batch, (int64_t)n_heads,
                                              (int64_t)n_kv, (int64_t)seq_len, (int64_t)head_dim));
    return;
  }
  finish("flash_attn_fwd",
         mi_flash_attn_fwd(get_stream(), Q, K, V, O, nullptr, (int64_t)batch, (int64_t)n_heads,
                           (int64_t)n_kv, (int64_t)seq_len, (int64_t)head_dim, 1, MI_ATTN_O_BHTD));
}

void cross_entropy(const void* logits, const uint32_t* targets, float* loss_out,
                   float* grad_logits, size_t total_tokens, size_t vocab_size) {
  if (total_tokens == 0 || vocab_size == 0) {  // MetalBridge.mm:1848
    t_status = MI_OK;
    return;
  }
  if (!ce_state(total_tokens)) {
    t_status = MI_ERR_HIP;
    std::fprintf(stderr, "[mi_bridge] cross_entropy: could not allocate the loss buffers\n");
    return;
  }
  if (t_in_scope && t_ce_n == CE_PENDING) {  // staging full: drain the scope's work once
    if (mi_stream_sync(get_stream()) != MI_OK) {
      finish("cross_entropy", MI_ERR_HIP);
      return;
    }
    ce_flush();
  }
  float* dev_loss = t_ce_dev + t_ce_rows;
  int st = mi_cross_entropy(get_stream(), logits, MI_BF16, (int64_t)vocab_size, targets,
                            (int64_t)total_tokens, (int64_t)vocab_size,
                            (float)(1.0 / (double)total_tokens), t_ce_dev, dev_loss, grad_logits,
                            MI_F32, (int64_t)vocab_size);
  if (st == MI_OK && loss_out) {
    if (hipMemcpyAsync(&t_ce_host[t_ce_n], dev_loss, sizeof(float), hipMemcpyDeviceToHost,
                       get_stream()) != hipSuccess) {
      t_status = MI_ERR_HIP;
      std::fprintf(stderr, "[mi_bridge] cross_entropy: loss copy failed\n");
      return;
    }
    t_ce_dst[t_ce_n++] = loss_out;
  }
  finish("cross_entropy", st);
  if (!t_in_scope && t_status == MI_OK) ce_flush();
}

void rms_norm_forward(const float* input, float* output, const float* weight, float eps,
                      size_t num_rows, size_t dims) {
  finish("rms_norm_forward",
         mi_rmsnorm_fwd(get_stream(), (void*)input, nullptr, weight, MI_BF16, output, nullptr,
                        (int64_t)num_rows, (int64_t)dims, (int64_t)dims, MI_BF16, eps));
}

void rms_norm_backward(const float* grad_output, const float* input, const float* weight,
                       float* grad_input, float* grad_weight, float eps, size_t num_rows,
                       size_t dims) {
  size_t ws_bytes = 0;
  void* ws = grad_weight ? grow_workspace(mi_rmsnorm_bwd_workspace_size((int64_t)num_rows, (int64_t)dims),
                                          &ws_bytes)
                         : nullptr;
  finish("rms_norm_backward",
         mi_rmsnorm_bwd(get_stream(), grad_output, input, weight, MI_BF16, nullptr, grad_input,
                        grad_weight, MI_BF16, 0.0f, (int64_t)num_rows, (int64_t)dims, (int64_t)dims,
                        MI_BF16, eps, ws, ws_bytes));
}

void fused_add_norm(float* x_residual, const float* residual, const float* weight, float* output,
                    size_t num_rows, size_t D, float eps) {
  finish("fused_add_norm",
         mi_rmsnorm_fwd(get_stream(), x_residual, residual, weight, MI_F32, output, nullptr,
                        (int64_t)num_rows, (int64_t)D, (int64_t)D, MI_F32, eps));
}

namespace {
// W' (the norm weight folded into the projection) and 1/rms per row for fused_norm_matmul.
thread_local void* t_fold = nullptr;
thread_local size_t t_fold_bytes = 0;

bool fold_state(size_t bytes) {
  if (bytes <= t_fold_bytes) return true;
  if (t_fold) {
    if (hipStreamSynchronize(get_stream()) != hipSuccess) return false;
    (void)hipFree(t_fold);
  }
  t_fold = nullptr;
  t_fold_bytes = 0;
  if (hipMalloc(&t_fold, bytes) != hipSuccess) return false;
  t_fold_bytes = bytes;
  return true;
}
}  // namespace

void fused_norm_matmul(void* x, const void* residual, const float* norm_weight, const void* W, void* out,
                       size_t rows, size_t dims, size_t N, float eps) {
  if (rows == 0 || dims == 0 || N == 0) {
    t_status = MI_OK;
    return;
  }
  const size_t wb = (dims * N * 2 + 255) / 256 * 256;
  if (!fold_state(wb + rows * sizeof(float))) {
    t_status = MI_ERR_HIP;
    std::fprintf(stderr, "[mi_bridge] fused_norm_matmul: could not allocate the folded weight\n");
    return;
  }
  void* Wf = t_fold;
  float* rstd = (float*)((char*)t_fold + wb);
  hipStream_t st = get_stream();
  int s = mi_rmsnorm_fwd(st, x, residual, norm_weight, MI_F32, nullptr, rstd, (int64_t)rows, (int64_t)dims,
                         (int64_t)dims, MI_BF16, eps);
  if (s == MI_OK)
    s = mi_rmsnorm_fold_weight(st, norm_weight, MI_F32, W, (int64_t)N, (int64_t)dims, (int64_t)N, MI_BF16, Wf,
                               (int64_t)N);
  size_t wsb = 0;
  void* ws = s == MI_OK ? workspace_for(0, 0, rows, N, dims, MI_BF16, MI_BF16, &wsb) : nullptr;
  mi_epilogue e;
  std::memset(&e, 0, sizeof(e));
  e.row_scale = rstd;
  if (s == MI_OK)
    s = mi_gemm(st, 0, 0, (int64_t)rows, (int64_t)N, (int64_t)dims, 1.0f, x, (int64_t)dims, Wf, (int64_t)N,
                MI_BF16, 0.0f, out, (int64_t)N, MI_BF16, &e, ws, wsb);
  finish("fused_norm_matmul", s);
}

void fused_backward_add_norm(const void* grad_output, const void* input, const void* weight,
                             const void* residual, void* grad_input, size_t num_rows, size_t D,
                             float eps) {
  finish("fused_backward_add_norm",
         mi_rmsnorm_bwd(get_stream(), grad_output, input, weight, MI_F32, residual, grad_input,
                        nullptr, MI_F32, 0.0f, (int64_t)num_rows, (int64_t)D, (int64_t)D, MI_BF16,
                        eps, nullptr, 0));
}

void fused_attn_bwd(const void* Q, const void* K, const void* V, const void* dO, void* dQ,
                    void* dK, void* dV, size_t batch, size_t n_heads, size_t n_kv,
                    size_t seq_len, size_t head_dim) {
  const size_t rows = batch * n_heads * seq_len;
  if (rows == 0 || head_dim == 0) {
    t_status = MI_OK;
    return;
  }
  const size_t kd = fused_dim(head_dim);
  if (kd && kd != head_dim) {
    if (n_kv == 0 || n_heads % n_kv) {
      finish("fused_attn_bwd", MI_ERR_SHAPE);
      return;
    }
    const size_t rq = rows, rk = batch * n_kv * seq_len;
    Padded b;
    if (!padded_buffers(rq, rk, kd, true, &b) || !attention_state(256, rows)) {
      t_status = MI_ERR_HIP;
      std::fprintf(stderr, "[mi_bridge] fused_attn_bwd: could not allocate the padded operands\n");
      return;
    }
    const float scale = (float)(1.0 / std::sqrt((double)head_dim));
    float* lse = t_att_f;
    float* delta = t_att_f + t_att_rows;
    int st = widen(Q, b.q, rq, head_dim, kd);
    if (st == MI_OK) st = widen(K, b.k, rk, head_dim, kd);
    if (st == MI_OK) st = widen(V, b.v, rk, head_dim, kd);
    if (st == MI_OK) st = widen(dO, b.dout, rq, head_dim, kd);
    if (st == MI_OK)
      st = mi_flash_attn_fwd_scaled(get_stream(), b.q, b.k, b.v, b.o, lse, (int64_t)batch, (int64_t)n_heads,
                                    (int64_t)n_kv, (int64_t)seq_len, (int64_t)kd, 1, MI_ATTN_O_BHTD, scale);
    const size_t ws = mi_flash_attn_bwd_workspace_size((int64_t)batch, (int64_t)n_heads, (int64_t)seq_len);
    const bool have_ws = ws && sp_state(ws);
    if (st == MI_OK)
      st = mi_flash_attn_bwd_scaled(get_stream(), b.q, b.k, b.v, b.o, b.dout, lse, b.dq, b.dk, b.dv, delta,
                                    (int64_t)batch, (int64_t)n_heads, (int64_t)n_kv, (int64_t)seq_len,
                                    (int64_t)kd, 1, MI_ATTN_O_BHTD, have_ws ? t_sp : nullptr,
                                    have_ws ? t_sp_bytes : 0, scale);
    if (st == MI_OK) st = narrow(b.dq, dQ, rq, head_dim, kd);
    if (st == MI_OK) st = narrow(b.dk, dK, rk, head_dim, kd);
    if (st == MI_OK) st = narrow(b.dv, dV, rk, head_dim, kd);
    finish("fused_attn_bwd", st);
    return;
  }
  if (!kd) {
    if (n_kv == 0 || n_heads % n_kv) {
      finish("fused_attn_bwd", MI_ERR_SHAPE);
      return;
    }
    finish("fused_attn_bwd", materialised_bwd(Q, K, V, dO, dQ, dK, dV, (int64_t)batch, (int64_t)n_heads,
                                              (int64_t)n_kv, (int64_t)seq_len, (int64_t)head_dim));
    return;
  }
  if (!attention_state(rows * head_dim * 2, rows)) {
    t_status = MI_ERR_HIP;
    std::fprintf(stderr, "[mi_bridge] fused_attn_bwd: could not allocate the forward state\n");
    return;
  }
  float* lse = t_att_f;
  float* delta = t_att_f + t_att_rows;
  int st = mi_flash_attn_fwd(get_stream(), Q, K, V, t_att_o, lse, (int64_t)batch, (int64_t)n_heads,
                             (int64_t)n_kv, (int64_t)seq_len, (int64_t)head_dim, 1, MI_ATTN_O_BHTD);
  // dS^T workspace (bridge-owned, shared with the materialised path's S/P buffer)
  const size_t ws = mi_flash_attn_bwd_workspace_size((int64_t)batch, (int64_t)n_heads, (int64_t)seq_len);
  const bool have_ws = ws && sp_state(ws);
  if (st == MI_OK)
    st = mi_flash_attn_bwd(get_stream(), Q, K, V, t_att_o, dO, lse, dQ, dK, dV, delta,
                           (int64_t)batch, (int64_t)n_heads, (int64_t)n_kv, (int64_t)seq_len,
                           (int64_t)head_dim, 1, MI_ATTN_O_BHTD, have_ws ? t_sp : nullptr,
                           have_ws ? t_sp_bytes : 0);
  finish("fused_attn_bwd", st);
}

void residual_add(float* a, const float* b, size_t n) {
  finish("residual_add", mi_residual_add(get_stream(), a, b, (int64_t)n, MI_BF16));
}

void residual_add_f32(float* a, const float* b, size_t n) {
  finish("residual_add_f32", mi_residual_add(get_stream(), a, b, (int64_t)n, MI_F32));
}

std::vector<size_t> matmul_shape(const DeviceTensor& a, const DeviceTensor& b) {
  const size_t ra = a.shape.size(), rb = b.shape.size();
  if (ra < 2 || rb < 2) throw std::invalid_argument("Matmul requires at least 2 dimensions");
  if (rb == 2 && ra != 2) {
    if (a.shape.back() != b.shape[0])
      throw std::invalid_argument("Inner dimensions must match for projection");
    std::vector<size_t> s = a.shape;
    s.back() = b.shape[1];
    return s;
  }
  if (ra != rb) throw std::invalid_argument("Batch size must match for matrix multiplication");
  for (size_t i = 0; i + 2 < ra; ++i)
    if (a.shape[i] != b.shape[i])
      throw std::invalid_argument("Batch dimension must match for matmul");
  if (a.shape[ra - 1] != b.shape[rb - 2])
    throw std::invalid_argument("Inner dimensions must match for matmul");
  std::vector<size_t> s = a.shape;
  s.back() = b.shape.back();
  return s;
}

void matmul(const DeviceTensor& a, const DeviceTensor& b, DeviceTensor& out) {
  const std::vector<size_t> s = matmul_shape(a, b);
  if (a.dtype != b.dtype) throw std::invalid_argument("Matmul operands must share a dtype");
  out.shape = s;
  out.dtype = a.dtype;
  const int dt = a.dtype == DType::BF16 ? MI_BF16 : MI_F32;
  const size_t ra = a.shape.size();
  int st;
  if (b.shape.size() == 2 && ra != 2) {
    size_t M = 1;
    for (size_t i = 0; i + 1 < ra; ++i) M *= a.shape[i];
    const size_t K = a.shape.back(), N = b.shape[1];
    size_t ws_bytes = 0;
    void* ws = workspace_for(0, 0, M, N, K, dt, dt, &ws_bytes);
    st = mi_gemm(get_stream(), 0, 0, (int64_t)M, (int64_t)N, (int64_t)K, 1.0f, a.data, (int64_t)K,
                 b.data, (int64_t)N, dt, 0.0f, out.data, (int64_t)N, dt, nullptr, ws, ws_bytes);
  } else {
    size_t nb = 1;
    for (size_t i = 0; i + 2 < ra; ++i) nb *= a.shape[i];
    const size_t M = a.shape[ra - 2], K = a.shape[ra - 1], N = b.shape.back();
    mi_batch bt;
    std::memset(&bt, 0, sizeof(bt));
    bt.batch = (int64_t)nb;
    bt.heads = 1;
    bt.a_outer = (int64_t)(M * K);
    bt.b_outer = (int64_t)(K * N);
    bt.c_outer = (int64_t)(M * N);
    bt.a_group = bt.b_group = bt.c_group = 1;
    bt.k_segments = 1;
    st = mi_gemm_batched(get_stream(), 0, 0, (int64_t)M, (int64_t)N, (int64_t)K, 1.0f, a.data,
                         (int64_t)K, b.data, (int64_t)N, dt, 0.0f, out.data, (int64_t)N, dt, &bt,
                         nullptr, nullptr, 0);
  }
  if (st != MI_OK) throw std::runtime_error(std::string("mi_gemm: ") + mi_last_error());
  finish("matmul", st);
}

// ---- GEMM profiler -------------------------------------------------------------

GemmProfiler& GemmProfiler::instance() {
  static GemmProfiler p;
  return p;
}

void GemmProfiler::enable(bool on) { (void)mi_profiler_enable(on ? 1 : 0); }

void GemmProfiler::begin_step() {
  if (mi_profiler_begin_step() != MI_OK)
    std::fprintf(stderr, "[mi_bridge] GemmProfiler::begin_step: %s\n", mi_last_error());
}

std::vector<GemmRecord> GemmProfiler::records() const {
  std::vector<GemmRecord> out;
  const int64_t n = mi_profiler_count();
  for (int64_t i = 0; i < n; ++i) {
    mi_gemm_record r;
    if (mi_profiler_record(i, &r) != MI_OK) {
      std::fprintf(stderr, "[mi_bridge] GemmProfiler::records: %s\n", mi_last_error());
      break;
    }
    out.push_back(GemmRecord{(size_t)r.M, (size_t)r.N, (size_t)r.K, r.transA != 0, r.transB != 0,
                             r.gpu_ms, r.kernel, (size_t)r.batch});
  }
  return out;
}

const char* GemmProfiler::op_name(size_t M, size_t N, size_t K, bool tA, bool tB) {
  (void)M; (void)N; (void)K;
  if (!tA && !tB) return "forward (NN)";
  if (!tA && tB) return "input gradient (NT)";
  if (tA && !tB) return "weight gradient (TN)";
  return "TT";
}

void GemmProfiler::print_summary(double step_gpu_ms) const {
  struct Agg {
    size_t M, N, K;
    bool tA, tB;
    std::string kernel;
    double ms = 0.0, flop = 0.0;
    int calls = 0;
  };
  std::vector<Agg> agg;
  const std::vector<GemmRecord> recs = records();
  for (const GemmRecord& r : recs) {
    Agg* a = nullptr;
    for (Agg& x : agg)
      if (x.M == r.M && x.N == r.N && x.K == r.K && x.tA == r.transA && x.tB == r.transB) a = &x;
    if (!a) {
      agg.push_back(Agg{r.M, r.N, r.K, r.transA, r.transB, r.kernel});
      a = &agg.back();
    }
    a->ms += r.elapsed_ms;
    a->flop += 2.0 * r.M * r.N * r.K * r.batch;
    a->calls += 1;
  }
  std::sort(agg.begin(), agg.end(), [](const Agg& x, const Agg& y) { return x.ms > y.ms; });
  double total = 0.0;
  for (const Agg& a : agg) total += a.ms;
  std::printf("GEMM PROFILER  (step GPU time %.3f ms, GEMM GPU time %.3f ms)\n", step_gpu_ms, total);
  std::printf("%-22s %6s %6s %6s %5s %10s %9s  %s\n", "operation", "M", "N", "K", "calls", "GPU ms",
              "TFLOP/s", "kernel");
  for (const Agg& a : agg) {
    const double tflops = a.ms > 0 ? a.flop / (a.ms * 1e-3) / 1e12 : 0.0;
    std::printf("%-22s %6zu %6zu %6zu %5d %10.4f %9.1f  %s\n", op_name(a.M, a.N, a.K, a.tA, a.tB),
                a.M, a.N, a.K, a.calls, a.ms, tflops, a.kernel.c_str());
  }
  std::printf("%-22s %6s %6s %6s %5zu %10.4f\n", "TOTAL", "", "", "", recs.size(), total);
  std::fflush(stdout);
}

double accum_gpu_time_ms() {
  double ms = 0.0;
  int64_t n = 0;
  (void)mi_profiler_totals(&ms, &n);
  return ms;
}

size_t count_gpu_calls() {
  double ms = 0.0;
  int64_t n = 0;
  (void)mi_profiler_totals(&ms, &n);
  return (size_t)n;
}

void reset_profile_stats() { (void)mi_profiler_reset(); }

}  // namespace mi_bridge
