/*
 * mi_oracle.c -- CPU restatement of the reference engine's matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP GEMM core
 * is compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never links
 * or calls it, and no product code path falls back to it.
 *
 * Reference: rahul238xaviers/large-language-model, C++ engine under cpp/.
 * The reference's own CPU path (Accelerate cblas_sgemm, MetalBridge.mm:691-701)
 * is macOS-only and cannot be compiled on Linux, so this is a restatement of
 * its semantics with float64 accumulation:
 *
 *   mo_gemm_ex     C = alpha*op(A)*op(B) [+ bias] [+ beta*C0] [+ R]
 *                  op(A)[m,k] = tA ? A[k*lda+m] : A[m*lda+k]   (gemm_bf16.metal:45)
 *                  op(B)[k,n] = tB ? B[n*ldb+k] : B[k*ldb+n]   (gemm_bf16.metal:63)
 *                  alpha=1, beta=0 is cblas_sgemm as called at MetalBridge.mm:695-697;
 *                  beta=1 is the accumulating dW epilogue of gemm_backward.metal:104-115
 *                  and Transformer.cpp:236,288-289; R is residual_add.metal:27
 *                  (a[i] += b[i]) fused as an epilogue.  The bias row-broadcast has no
 *                  reference counterpart (the engine has no linear bias) and is
 *                  pinned by its closed form only.
 *                  mode 1 (dual-B):  C = SiLU(alpha*A*Bg) * (alpha*A*Bu)  (gemm_ffn.metal:160-181)
 *                  mode 2 (prologue): op(A) := SiLU(G)*U elementwise before the
 *                  product (fused_swiglu_gemm.metal:48-77); SiLU(x) = x/(1+exp(-x))
 *                  (Activations.cpp:31-75).
 *                  K is split into nseg segments of Kseg; segment j of A/B starts
 *                  at +j*segA / +j*segB.  This is how the GQA KV-group reduction
 *                  (Attention.cpp:332,344-345: the += over the nH/nKV query heads
 *                  sharing one kv head) is expressed as one long K loop.
 *   mo_attention_fwd / mo_attention_bwd
 *                  Attention.cpp:236-280 (forward, causal, stable softmax, GQA map
 *                  kv_h = h / (nH/nKV)) and Attention.cpp:292-348 (backward).
 *   mo_cross_entropy
 *                  Loss.cpp:43-195 (CrossEntropyLoss forward and backward): softmax
 *                  with max subtraction, -log(max(p_target, 1e-15)), the logits
 *                  gradient (p - onehot) * scale and the mean loss.
 *   mo_rmsnorm_fwd / mo_rmsnorm_bwd
 *                  RMSNorm.cpp:40-180 (forward, backward with the weight gradient)
 *                  and the decoder layer's fused forms: residual add before the
 *                  norm (fused_add_norm, Transformer.cpp:150-158) and the residual
 *                  gradient added to dx (fused_backward_add_norm, Transformer.cpp:441-466).
 *   mo_sgemm_omp   fp32 cache-blocked OpenMP SGEMM with cblas_sgemm row-major
 *                  semantics -- the CPU baseline timed next to the GPU.
 *   bf16 helpers   Tensor.hpp:16-27 (truncating fp32->bf16, bf16->fp32) plus RNE.
 *   mo_fill_normal repo-owned SplitMix64 + Box-Muller generator (the reference's
 *                  std::mt19937 + std::normal_distribution is implementation
 *                  defined, test_gpu_kernels.cpp:53-60, so it is not reproduced).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- bf16 conversions (Tensor.hpp:16-27) ---------------------------------- */

/* Reference float_to_bf16: keep the upper 16 bits (round toward zero). */
uint16_t mo_f32_to_bf16_trunc(float v) {
  uint32_t b;
  memcpy(&b, &v, 4);
  return (uint16_t)(b >> 16);
}

/* Round-to-nearest-even, NaN kept quiet. */
uint16_t mo_f32_to_bf16_rne(float v) {
  uint32_t b;
  memcpy(&b, &v, 4);
  if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x40u);
  b += 0x7fffu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

float mo_bf16_to_f32(uint16_t h) {
  uint32_t b = (uint32_t)h << 16;
  float f;
  memcpy(&f, &b, 4);
  return f;
}

/* In-place rounding of an fp32 array to bf16-representable values. */
void mo_round_bf16(float* x, int64_t n, int rne) {
  for (int64_t i = 0; i < n; ++i)
    x[i] = mo_bf16_to_f32(rne ? mo_f32_to_bf16_rne(x[i]) : mo_f32_to_bf16_trunc(x[i]));
}

void mo_to_bf16(const float* x, uint16_t* out, int64_t n, int rne) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = rne ? mo_f32_to_bf16_rne(x[i]) : mo_f32_to_bf16_trunc(x[i]);
}

void mo_from_bf16(const uint16_t* h, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = mo_bf16_to_f32(h[i]);
}

/* ---- deterministic normal generator --------------------------------------- */

static uint64_t splitmix64(uint64_t* s) {
  uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

/* Element i depends only on (seed, i): pairs (2j, 2j+1) come from one
 * Box-Muller draw of stream position j, so any sub-range can be regenerated. */
void mo_fill_normal(float* out, int64_t n, uint64_t seed, double mean, double stddev) {
  const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
  for (int64_t j = 0; j < (n + 1) / 2; ++j) {
    uint64_t s = seed * 0x2545f4914f6cdd1dull + (uint64_t)j * 0x9e3779b97f4a7c15ull;
    uint64_t a = splitmix64(&s), b = splitmix64(&s);
    double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740993.0); /* (0,1] */
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);         /* [0,1) */
    double r = sqrt(-2.0 * log(u1));
    out[2 * j] = (float)(mean + stddev * r * cos(two_pi * u2));
    if (2 * j + 1 < n) out[2 * j + 1] = (float)(mean + stddev * r * sin(two_pi * u2));
  }
}

/* ---- general GEMM with epilogues ------------------------------------------ */

static inline double silu_d(double x) { return x / (1.0 + exp(-x)); }

/* op(A)[m, kk] for global reduction index kk = j*Kseg + k (segment j). */
static inline double opA(const float* A, const float* A2, int tA, int64_t lda, int64_t segA,
                         int64_t Kseg, int64_t m, int64_t kk, int mode) {
  int64_t j = kk / Kseg, k = kk % Kseg;
  int64_t off = j * segA + (tA ? k * lda + m : m * lda + k);
  if (mode == 2) return silu_d((double)A[off]) * (double)A2[off];
  return (double)A[off];
}

static inline double opB(const float* B, int tB, int64_t ldb, int64_t segB, int64_t Kseg,
                         int64_t kk, int64_t n) {
  int64_t j = kk / Kseg, k = kk % Kseg;
  return (double)B[j * segB + (tB ? n * ldb + k : k * ldb + n)];
}

/*
 * out[m*ldo+n] for m in rows (or all M when rows == NULL; then out row index = m,
 * otherwise out row index = position in rows[]).
 * mode: 0 plain, 1 dual-B SiLU gate (B2 = up weights), 2 SiLU-gate prologue on A (A2 = up).
 * C0 / bias / R may be NULL.
 */
void mo_gemm_ex(int tA, int tB, int64_t M, int64_t N, int64_t Kseg, int64_t nseg,
                int64_t segA, int64_t segB, double alpha,
                const float* A, int64_t lda, const float* A2,
                const float* B, int64_t ldb, const float* B2,
                double beta, const float* C0, int64_t ldc0,
                const float* bias, const float* R, int64_t ldr, int mode,
                double* out, int64_t ldo, const int64_t* rows, int64_t nrows) {
  const int64_t Ktot = Kseg * nseg;
  const int64_t nr = rows ? nrows : M;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t ri = 0; ri < nr; ++ri) {
    const int64_t m = rows ? rows[ri] : ri;
    double* arow = (double*)malloc(sizeof(double) * (size_t)(Ktot > 0 ? Ktot : 1));
    for (int64_t kk = 0; kk < Ktot; ++kk) arow[kk] = opA(A, A2, tA, lda, segA, Kseg, m, kk, mode);
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0, acc2 = 0.0;
      for (int64_t kk = 0; kk < Ktot; ++kk) {
        acc += arow[kk] * opB(B, tB, ldb, segB, Kseg, kk, n);
        if (mode == 1) acc2 += arow[kk] * opB(B2, tB, ldb, segB, Kseg, kk, n);
      }
      double t = (mode == 1) ? silu_d(alpha * acc) * (alpha * acc2) : alpha * acc;
      if (bias) t += (double)bias[n];
      if (beta != 0.0 && C0) t += beta * (double)C0[m * ldc0 + n];
      if (R) t += (double)R[m * ldr + n];
      out[ri * ldo + n] = t;
    }
    free(arow);
  }
}

void mo_gemm(int tA, int tB, int64_t M, int64_t N, int64_t K, double alpha,
             const float* A, int64_t lda, const float* B, int64_t ldb,
             double* out, int64_t ldo) {
  mo_gemm_ex(tA, tB, M, N, K, 1, 0, 0, alpha, A, lda, NULL, B, ldb, NULL, 0.0, NULL, 0,
             NULL, NULL, 0, 0, out, ldo, NULL, 0);
}

/* ---- GQA attention (Attention.cpp:236-280, 292-348) ------------------------ */

/*
 * Q4 [B,nH,T,d], K4/V4 [B,nKV,T,d] (reshape_to_4d, Attention.cpp:68-100).
 * O [B,T,nH*d] (Attention.cpp:270-278).  Optional P [B,nH,T,T] with zeros above
 * the diagonal (causal s_k <= s_q).  Everything in float64.
 */
void mo_attention_fwd(int64_t Bn, int64_t nH, int64_t nKV, int64_t T, int64_t d,
                      const float* Q4, const float* K4, const float* V4,
                      double* O, double* P) {
  const int64_t g = nH / nKV;
  const double scale = 1.0 / sqrt((double)d);
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int64_t b = 0; b < Bn; ++b)
    for (int64_t h = 0; h < nH; ++h) {
      const int64_t kvh = h / g;
      double* sc = (double*)malloc(sizeof(double) * (size_t)T);
      for (int64_t q = 0; q < T; ++q) {
        const float* qr = Q4 + ((b * nH + h) * T + q) * d;
        double mx = -INFINITY;
        for (int64_t k = 0; k <= q; ++k) {
          const float* kr = K4 + ((b * nKV + kvh) * T + k) * d;
          double dot = 0.0;
          for (int64_t i = 0; i < d; ++i) dot += (double)qr[i] * (double)kr[i];
          sc[k] = dot * scale;
          if (sc[k] > mx) mx = sc[k];
        }
        double sum = 0.0;
        for (int64_t k = 0; k <= q; ++k) { sc[k] = exp(sc[k] - mx); sum += sc[k]; }
        double* orow = O + (b * T + q) * (nH * d) + h * d;
        for (int64_t i = 0; i < d; ++i) orow[i] = 0.0;
        for (int64_t k = 0; k <= q; ++k) {
          const double p = sc[k] / sum;
          if (P) P[((b * nH + h) * T + q) * T + k] = p;
          const float* vr = V4 + ((b * nKV + kvh) * T + k) * d;
          for (int64_t i = 0; i < d; ++i) orow[i] += p * (double)vr[i];
        }
        if (P)
          for (int64_t k = q + 1; k < T; ++k) P[((b * nH + h) * T + q) * T + k] = 0.0;
      }
      free(sc);
    }
}

/*
 * dO [B,T,nH*d] (grad_attn_output layout, Attention.cpp:321).  Outputs dQ4
 * [B,nH,T,d], dK4/dV4 [B,nKV,T,d] in float64 (zeroed here, then accumulated as
 * in Attention.cpp:332,344-345).  Parallel over (b, kv head) so the KV-group
 * accumulation stays race-free.
 */
void mo_attention_bwd(int64_t Bn, int64_t nH, int64_t nKV, int64_t T, int64_t d,
                      const float* Q4, const float* K4, const float* V4, const float* dO,
                      double* dQ, double* dK, double* dV) {
  const int64_t g = nH / nKV;
  const double scale = 1.0 / sqrt((double)d);
  memset(dQ, 0, sizeof(double) * (size_t)(Bn * nH * T * d));
  memset(dK, 0, sizeof(double) * (size_t)(Bn * nKV * T * d));
  memset(dV, 0, sizeof(double) * (size_t)(Bn * nKV * T * d));
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int64_t b = 0; b < Bn; ++b)
    for (int64_t kvh = 0; kvh < nKV; ++kvh) {
      double* p = (double*)malloc(sizeof(double) * (size_t)T);
      double* dp = (double*)malloc(sizeof(double) * (size_t)T);
      for (int64_t h = kvh * g; h < (kvh + 1) * g; ++h)
        for (int64_t q = 0; q < T; ++q) {
          const float* qr = Q4 + ((b * nH + h) * T + q) * d;
          double mx = -INFINITY;
          for (int64_t k = 0; k <= q; ++k) {
            const float* kr = K4 + ((b * nKV + kvh) * T + k) * d;
            double dot = 0.0;
            for (int64_t i = 0; i < d; ++i) dot += (double)qr[i] * (double)kr[i];
            p[k] = dot * scale;
            if (p[k] > mx) mx = p[k];
          }
          double sum = 0.0;
          for (int64_t k = 0; k <= q; ++k) sum += exp(p[k] - mx);
          for (int64_t k = 0; k <= q; ++k) p[k] = exp(p[k] - mx) / sum;
          const float* gr = dO + (b * T + q) * (nH * d) + h * d;
          double sdp = 0.0;
          for (int64_t k = 0; k <= q; ++k) {
            const float* vr = V4 + ((b * nKV + kvh) * T + k) * d;
            double* dvr = dV + ((b * nKV + kvh) * T + k) * d;
            double dot = 0.0;
            for (int64_t i = 0; i < d; ++i) {
              dot += (double)gr[i] * (double)vr[i];
              dvr[i] += p[k] * (double)gr[i];
            }
            dp[k] = dot;
            sdp += dot * p[k];
          }
          double* dqr = dQ + ((b * nH + h) * T + q) * d;
          for (int64_t k = 0; k <= q; ++k) {
            const double ds = p[k] * (dp[k] - sdp) * scale;
            const float* kr = K4 + ((b * nKV + kvh) * T + k) * d;
            double* dkr = dK + ((b * nKV + kvh) * T + k) * d;
            for (int64_t i = 0; i < d; ++i) {
              dqr[i] += ds * (double)kr[i];
              dkr[i] += ds * (double)qr[i];
            }
          }
        }
      free(p);
      free(dp);
    }
}

/*
 * Loss.cpp:43-195 in float64.  Per row r (token) with target y = targets[r]:
 * m = max_v x[v] (Loss.cpp:95-101), s = sum_v exp(x[v] - m) (:103-107),
 * p[v] = exp(x[v] - m) / s (:109-112), row_loss[r] = -log(max(p[y], 1e-15f))
 * (:114-116), grad[r*vocab + v] = (p[v] - [v == y]) * scale (:160, :182-186;
 * the reference's scale is 1 / (batch*seq_len)).  Returns scale * sum_r
 * row_loss[r] (:128-132).  grad may be NULL.  A target outside [0, vocab)
 * gives a NaN row loss and no one-hot term.
 */
double mo_cross_entropy(const float* logits, int64_t ld, const int64_t* targets, int64_t rows,
                        int64_t vocab, double scale, double* row_loss, double* grad) {
  const double floor_p = (double)1e-15f;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = logits + r * ld;
    double m = -INFINITY;
    for (int64_t v = 0; v < vocab; ++v)
      if ((double)x[v] > m) m = (double)x[v];
    double sum = 0.0;
    for (int64_t v = 0; v < vocab; ++v) sum += exp((double)x[v] - m);
    const int64_t y = targets[r];
    const int valid = y >= 0 && y < vocab;
    if (valid) {
      const double py = exp((double)x[y] - m) / sum;
      row_loss[r] = -log(py > floor_p ? py : floor_p);
      if (py != py) row_loss[r] = py;  /* NaN stays NaN, as std::max keeps it */
    } else {
      row_loss[r] = NAN;
    }
    if (grad)
      for (int64_t v = 0; v < vocab; ++v)
        grad[r * vocab + v] = (exp((double)x[v] - m) / sum - (valid && v == y ? 1.0 : 0.0)) * scale;
  }
  double total = 0.0;
  for (int64_t r = 0; r < rows; ++r) total += row_loss[r];
  return total * scale;
}

/*
 * RMSNorm forward in float64 (RMSNorm.cpp:40-75): per row, with r given, first
 * x := x + r stored back in x's dtype (round_bf16: RNE to bf16, the storage of
 * the bf16 path; Transformer.cpp:150-158 writes h back for the backward), then
 * rms = sqrt(sum x^2 / dims + eps), y = x / rms * w, rstd[row] = 1 / rms.
 */
void mo_rmsnorm_fwd(float* x, const float* r, const float* w, int64_t rows, int64_t dims,
                    double eps, int round_bf16, double* y, double* rstd) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows; ++i) {
    float* xr = x + i * dims;
    double ss = 0.0;
    for (int64_t c = 0; c < dims; ++c) {
      if (r) {
        float v = xr[c] + r[i * dims + c];
        if (round_bf16) v = mo_bf16_to_f32(mo_f32_to_bf16_rne(v));
        xr[c] = v;
      }
      ss += (double)xr[c] * (double)xr[c];
    }
    const double rms = sqrt(ss / (double)dims + eps);
    for (int64_t c = 0; c < dims; ++c) y[i * dims + c] = (double)xr[c] / rms * (double)w[c];
    if (rstd) rstd[i] = 1.0 / rms;
  }
}

/*
 * RMSNorm backward in float64 (RMSNorm.cpp:77-180): xhat = x / rms,
 * dx = (1/rms) * (dy*w - xhat * mean(dy*w*xhat)) (:137-160), plus rg when given
 * (fused_backward_add_norm.metal, Transformer.cpp:449-452: grad_h += grad_output);
 * dw += sum over rows of dy * xhat (:163-176, accumulated as the CPU path does).
 */
void mo_rmsnorm_bwd(const float* dy, const float* x, const float* w, const float* rg,
                    int64_t rows, int64_t dims, double eps, double* dx, double* dw) {
  for (int64_t i = 0; i < rows; ++i) {
    const float* xr = x + i * dims;
    const float* gr = dy + i * dims;
    double ss = 0.0;
    for (int64_t c = 0; c < dims; ++c) ss += (double)xr[c] * (double)xr[c];
    const double rms = sqrt(ss / (double)dims + eps);
    double s = 0.0;
    for (int64_t c = 0; c < dims; ++c) s += (double)gr[c] * (double)w[c] * ((double)xr[c] / rms);
    s /= (double)dims;
    for (int64_t c = 0; c < dims; ++c) {
      const double xhat = (double)xr[c] / rms;
      dx[i * dims + c] = (1.0 / rms) * ((double)gr[c] * (double)w[c] - xhat * s) +
                         (rg ? (double)rg[i * dims + c] : 0.0);
      if (dw) dw[c] += (double)gr[c] * xhat;
    }
  }
}

/* ---- fp32 CPU SGEMM baseline (cblas_sgemm semantics, MetalBridge.mm:695-697) -- */

/*
 * C = alpha*op(A)*op(B) + beta*C, row-major, fp32 throughout.  op(A) and op(B)
 * are packed into K-contiguous panels, then a register-blocked 4x16 kernel
 * runs over 64x256 output blocks in parallel.  Uses every thread OpenMP gives it.
 */
#define SG_MB 64
#define SG_NB 256
#define SG_KB 256
void mo_sgemm_omp(int tA, int tB, int64_t M, int64_t N, int64_t K, float alpha,
                  const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                  float* C, int64_t ldc) {
  if (M <= 0 || N <= 0) return;
  const int64_t mb = (M + SG_MB - 1) / SG_MB, nb = (N + SG_NB - 1) / SG_NB;
#pragma omp parallel
  {
    float* ap = (float*)aligned_alloc(64, sizeof(float) * SG_MB * SG_KB);
    float* bp = (float*)aligned_alloc(64, sizeof(float) * SG_KB * SG_NB);
    float* cb = (float*)aligned_alloc(64, sizeof(float) * SG_MB * SG_NB);
#pragma omp for collapse(2) schedule(dynamic, 1)
    for (int64_t ib = 0; ib < mb; ++ib)
      for (int64_t jb = 0; jb < nb; ++jb) {
        const int64_t m0 = ib * SG_MB, n0 = jb * SG_NB;
        const int64_t mc = (M - m0 < SG_MB) ? M - m0 : SG_MB;
        const int64_t nc = (N - n0 < SG_NB) ? N - n0 : SG_NB;
        memset(cb, 0, sizeof(float) * SG_MB * SG_NB);
        for (int64_t k0 = 0; k0 < K; k0 += SG_KB) {
          const int64_t kc = (K - k0 < SG_KB) ? K - k0 : SG_KB;
          /* ap[i*kc + k] = op(A)[m0+i, k0+k];  bp[k*SG_NB + j] = op(B)[k0+k, n0+j] */
          for (int64_t i = 0; i < mc; ++i)
            for (int64_t k = 0; k < kc; ++k)
              ap[i * kc + k] = tA ? A[(k0 + k) * lda + m0 + i] : A[(m0 + i) * lda + k0 + k];
          for (int64_t k = 0; k < kc; ++k)
            for (int64_t j = 0; j < nc; ++j)
              bp[k * SG_NB + j] = tB ? B[(n0 + j) * ldb + k0 + k] : B[(k0 + k) * ldb + n0 + j];
          for (int64_t k = 0; k < kc; ++k)
            for (int64_t j = nc; j < SG_NB; ++j) bp[k * SG_NB + j] = 0.0f;
          for (int64_t i = 0; i < mc; ++i) {
            float* crow = cb + i * SG_NB;
            const float* arow = ap + i * kc;
            for (int64_t k = 0; k < kc; ++k) {
              const float a = arow[k];
              const float* brow = bp + k * SG_NB;
#pragma omp simd
              for (int64_t j = 0; j < SG_NB; ++j) crow[j] += a * brow[j];
            }
          }
        }
        for (int64_t i = 0; i < mc; ++i)
          for (int64_t j = 0; j < nc; ++j) {
            float* c = C + (m0 + i) * ldc + n0 + j;
            *c = alpha * cb[i * SG_NB + j] + (beta != 0.0f ? beta * *c : 0.0f);
          }
      }
    free(ap);
    free(bp);
    free(cb);
  }
}

int mo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
