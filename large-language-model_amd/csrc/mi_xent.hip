// mi_xent.hip -- softmax cross-entropy over rows of logits (the loss and the
// logits gradient after the LM head), gfx950.
//
// Reference: CrossEntropyLoss::forward / backward (cpp/src/Loss.cpp:43-195) and
// its GPU kernel cross_entropy.metal.  Per row (token) r with target y:
//   m = max_v x[v],  s = sum_v exp(x[v] - m),  p[v] = exp(x[v] - m) / s
//   loss_r  = -log(max(p[y], 1e-15))                          (Loss.cpp:112-115)
//   grad[v] = (p[v] - [v == y]) * scale   (scale = 1 / tokens, Loss.cpp:160,182-186)
// and the mean loss sum_r loss_r * scale (Loss.cpp:132).
//
// HBM-bound: one read of each logit and one write of each gradient element.
// One workgroup of 512 threads (8 waves) per row.
//   * Vector kernel: the row is loaded once into registers as 16-byte vectors
//     (up to 16 per thread: 65536 bf16 or 32768 fp32 logits), the max and the
//     sum of exponentials are block reductions over those registers, and the
//     gradient is written from them.  The row is read from HBM once, and the
//     gradient may overwrite the logits in place (every load of the row is
//     issued before the first barrier, every store after the second).
//   * Streaming kernel (longer rows, or rows that are not whole 16-byte
//     vectors): pass 1 keeps an online (max, sum) per thread, pass 2 re-reads
//     each element and writes its gradient; in place is safe too, as each
//     element is read and then written by one thread.
// Every reduction runs in a fixed order, so results are bit-identical across
// launches (the reference's atomic loss sum, cross_entropy.metal, is not).
//
// exp(x - m) is computed as 2^(x*log2(e) - m*log2(e)).  The loss is computed
// from the same exponent as the sum, loss = (log2(s) - a_y) * ln 2 with
// a_y = y's exponent, so the rounding of m*log2(e) cancels; it equals the
// reference's -log(max(p_y, 1e-15)) up to rounding, including the clamp at
// -log(1e-15).  NaN logits give NaN, as in the reference.  A target outside
// [0, vocab) gives a NaN loss and no one-hot term (the reference reads out of
// bounds there).
#include <hip/hip_runtime.h>
#include <math.h>

#include "mi_gemm_device.hpp"
#include "mi_xent.hpp"

namespace mig {
namespace {

constexpr float XENT_L2E = 1.4426950408889634f;
constexpr float XENT_LN2 = 0.6931471805599453f;
constexpr float XENT_LOSS_CLAMP = 34.538776394910684f;  // -log(1e-15)

typedef uint32_t xu32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t xu32x2_t __attribute__((ext_vector_type(2)));

template <bool BF16>
__device__ __forceinline__ float elem_of(const xu32x4_t& v, int e) {
  if constexpr (BF16)
    return (e & 1) ? __uint_as_float(v[e >> 1] & 0xffff0000u) : __uint_as_float(v[e >> 1] << 16);
  else
    return __uint_as_float(v[e]);
}

template <bool BF16>
__device__ __forceinline__ float load_elem(const void* row, int v) {
  if constexpr (BF16) return bf16_bits_to_f32(((const uint16_t*)row)[v]);
  else return ((const float*)row)[v];
}

template <bool BF16>
__device__ __forceinline__ void store_elem(void* row, int v, float g) {
  if constexpr (BF16) ((uint16_t*)row)[v] = (uint16_t)f32_to_bf16_rne(g);
  else ((float*)row)[v] = g;
}

// Butterfly reductions inside a wave.  Each step combines a value with its
// partner's by a commutative operation, so all 64 lanes end with the same bits.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Merge two partial softmax denominators (m, s), s = sum of exp(x - m) over a
// part of the row with maximum m.  A part with m = -inf holds no element.
__device__ __forceinline__ void merge_ms(float& m, float& s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  const float a = (m == -INFINITY) ? 0.0f : s * __builtin_amdgcn_exp2f((m - M) * XENT_L2E);
  const float b = (m2 == -INFINITY) ? 0.0f : s2 * __builtin_amdgcn_exp2f((m2 - M) * XENT_L2E);
  m = M;
  s = a + b;
}

__device__ __forceinline__ float clamp_loss(float l) { return l > XENT_LOSS_CLAMP ? XENT_LOSS_CLAMP : l; }

template <bool IN_BF16, bool OUT_BF16, int NV>
__global__ void __launch_bounds__(XENT_THREADS) xent_vec_kernel(XentParams p) {
  constexpr int EV = IN_BF16 ? 8 : 4;  // elements per 16-byte vector
  constexpr int NW = XENT_THREADS / 64;
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nvec = p.vocab / EV;
  const char* lrow = (const char*)p.logits + (int64_t)row * p.ld * (IN_BF16 ? 2 : 4);
  const uint32_t y = p.targets[row];
  // y's logit is read before the first barrier: after the second one other
  // threads may be overwriting the row with its gradient.
  float xy = 0.0f;
  if (tid == 0 && y < (uint32_t)p.vocab) xy = load_elem<IN_BF16>(lrow, (int)y);

  // Slots past the row end hold -inf: no effect on the max, exp gives 0.
  const uint32_t NEG_INF = IN_BF16 ? 0xff80ff80u : 0xff800000u;
  xu32x4_t v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int j = tid + i * XENT_THREADS;
    v[i] = j < nvec ? *(const xu32x4_t*)(lrow + (int64_t)j * 16)
                    : xu32x4_t{NEG_INF, NEG_INF, NEG_INF, NEG_INF};
  }

  __shared__ float red_m[NW], red_s[NW];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < EV; ++e) mx = fmaxf(mx, elem_of<IN_BF16>(v[i], e));
  mx = wave_max(mx);
  if (lane == 0) red_m[wave] = mx;
  __syncthreads();
  float m = red_m[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) m = fmaxf(m, red_m[w]);
  const float mneg = -m * XENT_L2E;

  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < EV; ++e)
      s += __builtin_amdgcn_exp2f(__builtin_fmaf(elem_of<IN_BF16>(v[i], e), XENT_L2E, mneg));
  s = wave_sum(s);
  if (lane == 0) red_s[wave] = s;
  __syncthreads();
  float ssum = red_s[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) ssum += red_s[w];

  if (tid == 0) {
    float loss = __builtin_nanf("");
    if (y < (uint32_t)p.vocab) {
      const float a = __builtin_fmaf(xy, XENT_L2E, mneg);
      loss = clamp_loss((log2f(ssum) - a) * XENT_LN2);
    }
    p.row_loss[row] = loss;
  }

  if (p.grad) {
    const float inv = p.scale / ssum;
    char* grow = (char*)p.grad + (int64_t)row * p.ldg * (OUT_BF16 ? 2 : 4);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int j = tid + i * XENT_THREADS;
      if (j < nvec) {
        float g[EV];
#pragma unroll
        for (int e = 0; e < EV; ++e)
          g[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(elem_of<IN_BF16>(v[i], e), XENT_L2E, mneg)) * inv;
        const uint32_t base = (uint32_t)j * EV;
        if (y - base < (uint32_t)EV) {
#pragma unroll
          for (int e = 0; e < EV; ++e)
            if (base + e == y) g[e] -= p.scale;
        }
        if constexpr (OUT_BF16) {
          if constexpr (EV == 8) {
            *(xu32x4_t*)(grow + (int64_t)base * 2) =
                xu32x4_t{pack_bf16x2(g[0], g[1]), pack_bf16x2(g[2], g[3]), pack_bf16x2(g[4], g[5]),
                         pack_bf16x2(g[6], g[7])};
          } else {
            *(xu32x2_t*)(grow + (int64_t)base * 2) = xu32x2_t{pack_bf16x2(g[0], g[1]), pack_bf16x2(g[2], g[3])};
          }
        } else {
#pragma unroll
          for (int h = 0; h < EV / 4; ++h)
            *(xu32x4_t*)(grow + ((int64_t)base + 4 * h) * 4) =
                xu32x4_t{__float_as_uint(g[4 * h]), __float_as_uint(g[4 * h + 1]),
                         __float_as_uint(g[4 * h + 2]), __float_as_uint(g[4 * h + 3])};
        }
      }
    }
  }
}

template <bool IN_BF16, bool OUT_BF16>
__global__ void __launch_bounds__(XENT_THREADS) xent_stream_kernel(XentParams p) {
  constexpr int NW = XENT_THREADS / 64;
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const char* lrow = (const char*)p.logits + (int64_t)row * p.ld * (IN_BF16 ? 2 : 4);
  const uint32_t y = p.targets[row];
  float xy = 0.0f;  // read before the barrier, as in the vector kernel
  if (tid == 0 && y < (uint32_t)p.vocab) xy = load_elem<IN_BF16>(lrow, (int)y);

  // Pass 1: online max and sum per thread (s is relative to m).
  float m = -INFINITY, s = 0.0f;
  for (int v = tid; v < p.vocab; v += XENT_THREADS) {
    const float x = load_elem<IN_BF16>(lrow, v);
    if (x > m) {
      s = (m == -INFINITY ? s * 0.0f : s * __builtin_amdgcn_exp2f((m - x) * XENT_L2E)) + 1.0f;  // keeps a NaN
      m = x;
    } else if (x != -INFINITY) {
      s += __builtin_amdgcn_exp2f((x - m) * XENT_L2E);  // NaN x propagates
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    merge_ms(m, s, m2, s2);
  }
  __shared__ float red_m[NW], red_s[NW];
  if (lane == 0) {
    red_m[wave] = m;
    red_s[wave] = s;
  }
  __syncthreads();
  float M = red_m[0], S = red_s[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) merge_ms(M, S, red_m[w], red_s[w]);

  if (tid == 0) {
    float loss = __builtin_nanf("");
    if (y < (uint32_t)p.vocab) {
      const float a = (xy - M) * XENT_L2E;
      loss = clamp_loss((log2f(S) - a) * XENT_LN2);
    }
    p.row_loss[row] = loss;
  }

  if (p.grad) {
    const float inv = p.scale / S;
    char* grow = (char*)p.grad + (int64_t)row * p.ldg * (OUT_BF16 ? 2 : 4);
    for (int v = tid; v < p.vocab; v += XENT_THREADS) {
      float g = __builtin_amdgcn_exp2f((load_elem<IN_BF16>(lrow, v) - M) * XENT_L2E) * inv;
      if ((uint32_t)v == y) g -= p.scale;
      store_elem<OUT_BF16>(grow, v, g);
    }
  }
}

__global__ void __launch_bounds__(1024) xent_mean_kernel(const float* row_loss, int rows, float scale,
                                                         float* loss_out) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float s = 0.0f;
  for (int i = tid; i < rows; i += 1024) s += row_loss[i];
  s = wave_sum(s);
  __shared__ float red[16];
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (tid == 0) {
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < 16; ++w) t += red[w];
    loss_out[0] = t * scale;
  }
}

// ---- vocabulary chunks ---------------------------------------------------------
// The LM head without a full logits buffer: chunk c holds columns [c0, c0 + n) of
// every row in L[rows][ldl] (bf16).  Pass 1 merges each chunk's (max, sum exp) into
// the row's running (m, s) in chunk order and records the target's logit when it
// lies in the chunk; the finish kernel turns (m, s, x_y) into the row loss and keeps
// m and scale/s; pass 2 overwrites each recomputed chunk with its gradient
// scale * (softmax - onehot).  Every merge runs in a fixed order (deterministic).
__global__ void __launch_bounds__(256) xent_chunk_stats_kernel(const uint16_t* L, int64_t ldl, int n, int c0,
                                                               const uint32_t* targets, float* run_m,
                                                               float* run_s, float* xy, int first) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint16_t* lrow = L + (int64_t)row * ldl;
  float m = -INFINITY, s = 0.0f;
  if ((n & 7) == 0 && (ldl & 7) == 0) {  // 16-byte vectors of 8 logits, one rescale per vector
    for (int v = tid * 8; v < n; v += 256 * 8) {
      const xu32x4_t q = *(const xu32x4_t*)(lrow + v);
      float x[8], mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] = elem_of<true>(q, e);
        mx = fmaxf(mx, x[e]);
      }
      if (mx > m) {
        s = m == -INFINITY ? s * 0.0f : s * __builtin_amdgcn_exp2f((m - mx) * XENT_L2E);  // keeps a NaN
        m = mx;
      }
      if (m != -INFINITY) {
        const float mneg = -m * XENT_L2E;
#pragma unroll
        for (int e = 0; e < 8; ++e) s += __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], XENT_L2E, mneg));
      } else {  // every logit so far is -inf or NaN (fmaxf skips NaN): add the NaNs
#pragma unroll
        for (int e = 0; e < 8; ++e) s += x[e] == -INFINITY ? 0.0f : x[e];
      }
    }
  } else {
    for (int v = tid; v < n; v += 256) {
      const float x = bf16_bits_to_f32(lrow[v]);
      if (x > m) {
        s = (m == -INFINITY ? s * 0.0f : s * __builtin_amdgcn_exp2f((m - x) * XENT_L2E)) + 1.0f;  // keeps a NaN
        m = x;
      } else if (x != -INFINITY) {
        s += __builtin_amdgcn_exp2f((x - m) * XENT_L2E);  // NaN x propagates
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    merge_ms(m, s, m2, s2);
  }
  __shared__ float red_m[4], red_s[4];
  if (lane == 0) {
    red_m[wave] = m;
    red_s[wave] = s;
  }
  __syncthreads();
  if (tid == 0) {
    float M = red_m[0], S = red_s[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) merge_ms(M, S, red_m[w], red_s[w]);
    if (!first) {  // the running part (earlier chunks) first, then this chunk
      float M0 = run_m[row], S0 = run_s[row];
      merge_ms(M0, S0, M, S);
      M = M0;
      S = S0;
    }
    run_m[row] = M;
    run_s[row] = S;
    const uint32_t y = targets[row];
    if (y - (uint32_t)c0 < (uint32_t)n) xy[row] = bf16_bits_to_f32(lrow[y - (uint32_t)c0]);
  }
}

// Row loss from the merged (m, s) and the target's logit; run_s becomes scale / s.
__global__ void __launch_bounds__(256) xent_chunk_finish_kernel(int rows, int vocab, const uint32_t* targets,
                                                                const float* run_m, float* run_s,
                                                                const float* xy, float scale, float* row_loss) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  const float M = run_m[r], S = run_s[r];
  float loss = __builtin_nanf("");
  if (targets[r] < (uint32_t)vocab) loss = clamp_loss((log2f(S) - (xy[r] - M) * XENT_L2E) * XENT_LN2);
  row_loss[r] = loss;
  run_s[r] = scale / S;
}

// Gradient of one chunk in place: L[r][v] = scale * (exp(x - m) / s - [c0 + v == y]).
__global__ void __launch_bounds__(256) xent_chunk_grad_kernel(uint16_t* L, int64_t ldl, int n, int c0,
                                                              const uint32_t* targets, const float* run_m,
                                                              const float* run_inv, float scale) {
  const int row = blockIdx.x;
  uint16_t* lrow = L + (int64_t)row * ldl;
  const float mneg = -run_m[row] * XENT_L2E, inv = run_inv[row];
  const uint32_t yc = targets[row] - (uint32_t)c0;  // the target's column in the chunk (or past n)
  const bool vec = (n & 7) == 0 && (ldl & 7) == 0;  // 16-byte rows of 8 logits
  if (vec) {
    for (int v = threadIdx.x * 8; v < n; v += 256 * 8) {
      xu32x4_t q = *(const xu32x4_t*)(lrow + v);
      float g[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        g[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(elem_of<true>(q, e), XENT_L2E, mneg)) * inv;
        if ((uint32_t)(v + e) == yc) g[e] -= scale;
      }
      *(xu32x4_t*)(lrow + v) = xu32x4_t{pack_bf16x2(g[0], g[1]), pack_bf16x2(g[2], g[3]),
                                        pack_bf16x2(g[4], g[5]), pack_bf16x2(g[6], g[7])};
    }
  } else {
    for (int v = threadIdx.x; v < n; v += 256) {
      float g = __builtin_amdgcn_exp2f(__builtin_fmaf(bf16_bits_to_f32(lrow[v]), XENT_L2E, mneg)) * inv;
      if ((uint32_t)v == yc) g -= scale;
      lrow[v] = (uint16_t)f32_to_bf16_rne(g);
    }
  }
}

template <bool IN_BF16, bool OUT_BF16>
hipError_t launch_vec(const XentParams& p, int nv, hipStream_t st) {
  const dim3 grid((unsigned)p.rows), block(XENT_THREADS);
  switch (nv) {
    case 1: hipLaunchKernelGGL((xent_vec_kernel<IN_BF16, OUT_BF16, 1>), grid, block, 0, st, p); break;
    case 2: hipLaunchKernelGGL((xent_vec_kernel<IN_BF16, OUT_BF16, 2>), grid, block, 0, st, p); break;
    case 4: hipLaunchKernelGGL((xent_vec_kernel<IN_BF16, OUT_BF16, 4>), grid, block, 0, st, p); break;
    case 8: hipLaunchKernelGGL((xent_vec_kernel<IN_BF16, OUT_BF16, 8>), grid, block, 0, st, p); break;
    default: hipLaunchKernelGGL((xent_vec_kernel<IN_BF16, OUT_BF16, 16>), grid, block, 0, st, p); break;
  }
  return hipGetLastError();
}

template <bool IN_BF16, bool OUT_BF16>
hipError_t launch_one(const XentParams& p, bool vector_path, hipStream_t st) {
  if (vector_path) {
    const int ev = IN_BF16 ? 8 : 4;
    const int per = (p.vocab / ev + XENT_THREADS - 1) / XENT_THREADS;
    const int nv = per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : 16;
    return launch_vec<IN_BF16, OUT_BF16>(p, nv, st);
  }
  hipLaunchKernelGGL((xent_stream_kernel<IN_BF16, OUT_BF16>), dim3((unsigned)p.rows), dim3(XENT_THREADS),
                     0, st, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_xent(const XentParams& p, bool in_bf16, bool out_bf16, bool vector_path,
                       hipStream_t stream) {
  if (in_bf16)
    return out_bf16 ? launch_one<true, true>(p, vector_path, stream)
                    : launch_one<true, false>(p, vector_path, stream);
  return out_bf16 ? launch_one<false, true>(p, vector_path, stream)
                  : launch_one<false, false>(p, vector_path, stream);
}

hipError_t launch_xent_chunk_stats(const void* L, int64_t ldl, int rows, int n, int c0,
                                   const uint32_t* targets, float* run_m, float* run_s, float* xy, bool first,
                                   hipStream_t stream) {
  hipLaunchKernelGGL(xent_chunk_stats_kernel, dim3((unsigned)rows), dim3(256), 0, stream, (const uint16_t*)L,
                     ldl, n, c0, targets, run_m, run_s, xy, first ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_xent_chunk_finish(int rows, int vocab, const uint32_t* targets, const float* run_m,
                                    float* run_s, const float* xy, float scale, float* row_loss,
                                    hipStream_t stream) {
  hipLaunchKernelGGL(xent_chunk_finish_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, rows,
                     vocab, targets, run_m, run_s, xy, scale, row_loss);
  return hipGetLastError();
}

hipError_t launch_xent_chunk_grad(void* L, int64_t ldl, int rows, int n, int c0, const uint32_t* targets,
                                  const float* run_m, const float* run_inv, float scale, hipStream_t stream) {
  hipLaunchKernelGGL(xent_chunk_grad_kernel, dim3((unsigned)rows), dim3(256), 0, stream, (uint16_t*)L, ldl, n,
                     c0, targets, run_m, run_inv, scale);
  return hipGetLastError();
}

hipError_t launch_xent_mean(const float* row_loss, int rows, float scale, float* loss_out,
                            hipStream_t stream) {
  hipLaunchKernelGGL(xent_mean_kernel, dim3(1), dim3(1024), 0, stream, row_loss, rows, scale, loss_out);
  return hipGetLastError();
}

}  // namespace mig
