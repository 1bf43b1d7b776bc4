// mi_norm.hip -- RMSNorm forward (optionally after a residual add) and backward
// (optionally plus a residual gradient, optionally with the weight gradient),
// gfx950.
//
// Reference (cpp/ of the engine): RMSNorm::forward / backward (src/RMSNorm.cpp:48-180),
// GPU kernels rms_norm_forward.metal, rms_norm_backward.metal, and the fused forms
// the decoder layer calls: fused_add_norm (h += r; y = rmsnorm(h), Transformer.cpp:150-158)
// and fused_backward_add_norm (dx = rmsnorm_backward(dy) + residual gradient,
// Transformer.cpp:441-466).  Per row of dims values, in fp32:
//   rms = sqrt(sum x^2 / dims + eps)
//   y   = (x / rms) * w                                   (RMSNorm.cpp:40-47)
//   dx  = (1/rms) * (dy*w - xhat * mean(dy*w*xhat)) [+ r], xhat = x / rms  (RMSNorm.cpp:137-160)
//   dw  = sum over rows of dy * xhat                       (RMSNorm.cpp:163-176)
// With a residual in the forward, x is first replaced by x + r in its own dtype (as
// the reference writes h back for the backward) and the norm uses the stored value.
//
// HBM-bound row kernels.  Register path: one wave per row, each lane holding up to
// 8 16-byte vectors of the row (4096 bf16 / 2048 fp32 values), reductions by
// butterflies inside the wave, no LDS and no barriers in the forward.  The backward
// runs a fixed grid of 4-wave workgroups over the rows, each lane accumulating the
// weight gradient of its own columns in registers; the waves of a workgroup add
// their partials in wave order through LDS into one workspace row, and a second
// kernel sums the workspace rows in order: dw is bit-identical across launches.
// Generic path (rows that are not whole aligned 16-byte vectors, or longer): one
// 256-thread workgroup per row, strided passes over global memory.  xhat is formed as
// x * (1/rms): one reciprocal per row instead of a division per element (the divide
// sequence made the backward VALU-bound).
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "mi_gemm_device.hpp"
#include "mi_norm.hpp"

namespace mig {
namespace {

typedef uint32_t nu32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t nu32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float nwave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;  // commutative steps: every lane holds the same bits
}

__device__ __forceinline__ float bf16_round(float v) { return bf16_bits_to_f32(f32_to_bf16_rne(v)); }

// One 16-byte vector of activations: 8 bf16 or 4 fp32 values at element e0.
template <bool BF16>
__device__ __forceinline__ void load_act(const char* row, int e0, float* v) {
  if constexpr (BF16) {
    const nu32x4_t q = *(const nu32x4_t*)(row + (int64_t)e0 * 2);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = __uint_as_float(q[k] << 16);
      v[2 * k + 1] = __uint_as_float(q[k] & 0xffff0000u);
    }
  } else {
    const nu32x4_t q = *(const nu32x4_t*)(row + (int64_t)e0 * 4);
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = __uint_as_float(q[k]);
  }
}

template <bool BF16>
__device__ __forceinline__ void store_act(char* row, int e0, const float* v) {
  if constexpr (BF16)
    *(nu32x4_t*)(row + (int64_t)e0 * 2) = nu32x4_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                    pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
  else
    *(nu32x4_t*)(row + (int64_t)e0 * 4) = nu32x4_t{__float_as_uint(v[0]), __float_as_uint(v[1]),
                                                   __float_as_uint(v[2]), __float_as_uint(v[3])};
}

// EV weight values at element e0 (EV = 8 for bf16 activations, 4 for fp32).
template <bool W_BF16, int EV>
__device__ __forceinline__ void load_w(const void* w, int e0, float* v) {
  if constexpr (W_BF16 && EV == 8) {
    load_act<true>((const char*)w, e0, v);
  } else if constexpr (W_BF16) {
    const nu32x2_t q = *(const nu32x2_t*)((const char*)w + (int64_t)e0 * 2);
    v[0] = __uint_as_float(q[0] << 16);
    v[1] = __uint_as_float(q[0] & 0xffff0000u);
    v[2] = __uint_as_float(q[1] << 16);
    v[3] = __uint_as_float(q[1] & 0xffff0000u);
  } else {
#pragma unroll
    for (int h = 0; h < EV / 4; ++h) load_act<false>((const char*)w, e0 + 4 * h, v + 4 * h);
  }
}

template <bool BF16>
__device__ __forceinline__ float ld_elem(const void* row, int c) {
  if constexpr (BF16) return bf16_bits_to_f32(((const uint16_t*)row)[c]);
  else return ((const float*)row)[c];
}

// Stores v at element c and returns the value as stored.
template <bool BF16>
__device__ __forceinline__ float st_elem(void* row, int c, float v) {
  if constexpr (BF16) {
    const uint32_t h = f32_to_bf16_rne(v);
    ((uint16_t*)row)[c] = (uint16_t)h;
    return bf16_bits_to_f32(h);
  } else {
    ((float*)row)[c] = v;
    return v;
  }
}

// Sum over a 256-thread workgroup, combined in wave order; red holds 4 floats.
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = nwave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();  // red is reused by the next reduction
  return t;
}

// ---- forward ----------------------------------------------------------------

template <bool BF16, bool W_BF16, int NV>
__global__ void __launch_bounds__(256) norm_fwd_vec(NormParams p) {
  constexpr int EV = BF16 ? 8 : 4, ES = BF16 ? 2 : 4;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;  // no barriers in this kernel
  const int nvec = p.dims / EV;
  char* xr = (char*)p.x + (int64_t)row * p.ld * ES;
  float v[NV][EV];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int j = lane + 64 * i;
    if (j < nvec) {
      load_act<BF16>(xr, j * EV, v[i]);
      if (p.r) {
        float rv[EV];
        load_act<BF16>((const char*)p.r + (int64_t)row * p.ld * ES, j * EV, rv);
#pragma unroll
        for (int e = 0; e < EV; ++e) v[i][e] += rv[e];
        store_act<BF16>(xr, j * EV, v[i]);
        if constexpr (BF16) {
#pragma unroll
          for (int e = 0; e < EV; ++e) v[i][e] = bf16_round(v[i][e]);  // the value stored
        }
      }
#pragma unroll
      for (int e = 0; e < EV; ++e) ss = __builtin_fmaf(v[i][e], v[i][e], ss);
    }
  }
  ss = nwave_sum(ss);
  const float rs = 1.0f / sqrtf(ss / (float)p.dims + p.eps);
  if (p.rstd && lane == 0) p.rstd[row] = rs;
  if (!p.y) return;  // statistic only (the norm folded into a GEMM)
  char* yr = (char*)p.y + (int64_t)row * p.ld * ES;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int j = lane + 64 * i;
    if (j < nvec) {
      float wv[EV], o[EV];
      load_w<W_BF16, EV>(p.w, j * EV, wv);
#pragma unroll
      for (int e = 0; e < EV; ++e) o[e] = v[i][e] * rs * wv[e];
      store_act<BF16>(yr, j * EV, o);
    }
  }
}

template <bool BF16, bool W_BF16>
__global__ void __launch_bounds__(256) norm_fwd_gen(NormParams p) {
  constexpr int ES = BF16 ? 2 : 4;
  __shared__ float red[4];
  const int row = blockIdx.x;
  char* xr = (char*)p.x + (int64_t)row * p.ld * ES;
  const char* rr = p.r ? (const char*)p.r + (int64_t)row * p.ld * ES : nullptr;
  char* yr = (char*)p.y + (int64_t)row * p.ld * ES;
  float ss = 0.0f;
  for (int c = threadIdx.x; c < p.dims; c += 256) {
    float v = ld_elem<BF16>(xr, c);
    if (rr) v = st_elem<BF16>(xr, c, v + ld_elem<BF16>(rr, c));
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = block_sum256(ss, red);
  const float rs = 1.0f / sqrtf(ss / (float)p.dims + p.eps);
  if (p.rstd && threadIdx.x == 0) p.rstd[row] = rs;
  if (!p.y) return;  // statistic only (the norm folded into a GEMM)
  for (int c = threadIdx.x; c < p.dims; c += 256)  // each thread re-reads what it wrote
    st_elem<BF16>(yr, c, ld_elem<BF16>(xr, c) * rs * ld_elem<W_BF16>(p.w, c));
}

// ---- backward ---------------------------------------------------------------

template <bool BF16>
__device__ __forceinline__ void unpack_act(nu32x4_t q, float* v) {
  if constexpr (BF16) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = __uint_as_float(q[k] << 16);
      v[2 * k + 1] = __uint_as_float(q[k] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = __uint_as_float(q[k]);
  }
}

// Sums of v and u over the 64 lanes of a wave, both chains interleaved.  Each step
// adds a lane's value to its partner's under an involution of the lane index (DPP
// swaps within a quad, the half-row and row mirrors, then lanes 16 and 32 apart), so
// partners add the same two values and every lane ends with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_partner(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, false));
}
__device__ __forceinline__ void nwave_sum2(float& v, float& u) {
  v += dpp_partner<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  u += dpp_partner<0xB1>(u);
  v += dpp_partner<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  u += dpp_partner<0x4E>(u);
  v += dpp_partner<0x141>(v);  // row_half_mirror: lane 7 - i within 8
  u += dpp_partner<0x141>(u);
  v += dpp_partner<0x140>(v);  // row_mirror: lane 15 - i within 16
  u += dpp_partner<0x140>(u);
  v += __shfl_xor(v, 16, 64);
  u += __shfl_xor(u, 16, 64);
  v += __shfl_xor(v, 32, 64);
  u += __shfl_xor(u, 32, 64);
}

// Each wave walks its rows with the next row's x, dy and residual gradient loaded
// (packed, 16-byte vectors) while the current row is computed, in two passes: (1)
// sum x^2 and dy*w*x, both reduced together; (2) dx = rinv*(dy*w) - rinv^3*t/dims*x
// + rg and the weight-gradient term dy*x*rinv.  The second pass unpacks the row again
// from a copy the compiler cannot see through, so the unpacked values of the first
// are not kept live.  The weight is unpacked once per kernel.  FULL: every lane owns
// NV whole vectors of each row (no bounds tests).
template <bool BF16, bool W_BF16, int NV, bool FULL>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NV <= 4 ? 2 : 1)))
    norm_bwd_vec(NormParams p) {
  constexpr int EV = BF16 ? 8 : 4, ES = BF16 ? 2 : 4;
  extern __shared__ float red_dw[];  // dims floats when p.dw
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nvec = p.dims / EV;
  const bool has_r = p.r != nullptr;
  auto live = [&](int i) __attribute__((always_inline)) { return FULL || lane + 64 * i < nvec; };
  float acc[NV][EV], wr[NV][EV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
#pragma unroll
    for (int e = 0; e < EV; ++e) acc[i][e] = wr[i][e] = 0.0f;
    if (live(i)) load_w<W_BF16, EV>(p.w, (lane + 64 * i) * EV, wr[i]);
  }
  const int stride = gridDim.x * 4;
  auto load_row = [&](int row, nu32x4_t* xq, nu32x4_t* gq, nu32x4_t* rq) __attribute__((always_inline)) {
    const int64_t off = (int64_t)row * p.ld * ES;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int j = lane + 64 * i;
      xq[i] = gq[i] = rq[i] = nu32x4_t{0u, 0u, 0u, 0u};
      if (live(i)) {
        xq[i] = *(const nu32x4_t*)((const char*)p.x + off + (int64_t)j * 16);
        gq[i] = *(const nu32x4_t*)((const char*)p.dy + off + (int64_t)j * 16);
        if (has_r) rq[i] = *(const nu32x4_t*)((const char*)p.r + off + (int64_t)j * 16);
      }
    }
  };
  nu32x4_t xq[NV], gq[NV], rq[NV];
  int row = blockIdx.x * 4 + wave;
  if (row < p.rows) load_row(row, xq, gq, rq);
  for (; row < p.rows; row += stride) {
    nu32x4_t xn[NV], gn[NV], rn[NV];
    if (row + stride < p.rows) load_row(row + stride, xn, gn, rn);
    float ss = 0.0f, t = 0.0f;  // sum x^2, sum dy*w*x (zeros past the row add nothing)
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float xv[EV], gv[EV];
      unpack_act<BF16>(xq[i], xv);
      unpack_act<BF16>(gq[i], gv);
#pragma unroll
      for (int e = 0; e < EV; ++e) {
        ss = __builtin_fmaf(xv[e], xv[e], ss);
        t = __builtin_fmaf(gv[e] * wr[i][e], xv[e], t);
      }
    }
    nwave_sum2(ss, t);
    const float rms = sqrtf(ss / (float)p.dims + p.eps);
    const float rinv = 1.0f / rms;
    const float cx = rinv * rinv * rinv * (t / (float)p.dims);  // rinv * (sum dy*w*xhat) / dims * rinv
    char* dxr = (char*)p.dx + (int64_t)row * p.ld * ES;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (live(i)) {
        nu32x4_t a = xq[i], b = gq[i];
        __asm__ volatile("" : "+v"(a), "+v"(b));
        float xv[EV], gv[EV], o[EV], rv[EV];
        unpack_act<BF16>(a, xv);
        unpack_act<BF16>(b, gv);
        unpack_act<BF16>(rq[i], rv);  // zeros without a residual gradient
#pragma unroll
        for (int e = 0; e < EV; ++e) {
          o[e] = __builtin_fmaf(rinv, gv[e] * wr[i][e], __builtin_fmaf(-cx, xv[e], rv[e]));
          acc[i][e] = __builtin_fmaf(gv[e] * rinv, xv[e], acc[i][e]);
        }
        store_act<BF16>(dxr, (lane + 64 * i) * EV, o);
      }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      xq[i] = xn[i];
      gq[i] = gn[i];
      rq[i] = rn[i];
    }
  }
  if (p.dw) {  // uniform: every thread takes it
    for (int w = 0; w < 4; ++w) {
      if (wave == w) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int j = lane + 64 * i;
          if (live(i)) {
#pragma unroll
            for (int e = 0; e < EV; ++e) {
              const int c = j * EV + e;
              red_dw[c] = (w == 0 ? 0.0f : red_dw[c]) + acc[i][e];
            }
          }
        }
      }
      __syncthreads();
    }
    float* wsr = p.ws + (int64_t)blockIdx.x * p.dims;
    for (int c = threadIdx.x; c < p.dims; c += 256) wsr[c] = red_dw[c];
  }
}

template <bool BF16, bool W_BF16>
__global__ void __launch_bounds__(256) norm_bwd_gen(NormParams p) {
  constexpr int ES = BF16 ? 2 : 4;
  __shared__ float red[4];
  float* wsr = p.dw ? p.ws + (int64_t)blockIdx.x * p.dims : nullptr;
  if (wsr)  // each thread owns columns tid + 256k of this workspace row
    for (int c = threadIdx.x; c < p.dims; c += 256) wsr[c] = 0.0f;
  for (int row = blockIdx.x; row < p.rows; row += gridDim.x) {
    const char* xr = (const char*)p.x + (int64_t)row * p.ld * ES;
    const char* gr = (const char*)p.dy + (int64_t)row * p.ld * ES;
    const char* rr = p.r ? (const char*)p.r + (int64_t)row * p.ld * ES : nullptr;
    char* dxr = (char*)p.dx + (int64_t)row * p.ld * ES;
    float ss = 0.0f;
    for (int c = threadIdx.x; c < p.dims; c += 256) {
      const float x = ld_elem<BF16>(xr, c);
      ss = __builtin_fmaf(x, x, ss);
    }
    ss = block_sum256(ss, red);
    const float rms = sqrtf(ss / (float)p.dims + p.eps);
    const float rinv = 1.0f / rms;
    float s2 = 0.0f;
    for (int c = threadIdx.x; c < p.dims; c += 256)
      s2 = __builtin_fmaf(ld_elem<BF16>(gr, c) * ld_elem<W_BF16>(p.w, c), ld_elem<BF16>(xr, c) * rinv, s2);
    s2 = block_sum256(s2, red) / (float)p.dims;  // its barriers order every read above before the writes below
    for (int c = threadIdx.x; c < p.dims; c += 256) {
      const float x = ld_elem<BF16>(xr, c), g = ld_elem<BF16>(gr, c);
      const float xhat = x * rinv;
      float o = rinv * (g * ld_elem<W_BF16>(p.w, c) - xhat * s2);
      if (rr) o += ld_elem<BF16>(rr, c);
      st_elem<BF16>(dxr, c, o);
      if (wsr) wsr[c] = __builtin_fmaf(g, xhat, wsr[c]);
    }
    __syncthreads();  // dx may alias dy or x: the next row's reads follow this row's writes
  }
}

// dw[c] = beta*dw[c] + sum_g ws[g][c].  One 1024-thread workgroup per 64 columns:
// lane = column, wave w sums rows w, w+16, ... (coalesced 256-byte rows, few
// loads per thread), then wave 0 adds the 16 wave sums in wave order.
template <bool DW_BF16>
__global__ void __launch_bounds__(1024) norm_dw_reduce(const float* ws, int G, int dims, float beta,
                                                       void* dw) {
  __shared__ float red[16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  float s = 0.0f;
  if (c < dims)
    for (int g0 = wave; g0 < G; g0 += 16 * 8) {  // 8 loads in flight, summed in g order
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int g = g0 + 16 * k;
        v[k] = g < G ? ws[(int64_t)g * dims + c] : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) s += v[k];
    }
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && c < dims) {
    float t = red[0][lane];
#pragma unroll
    for (int w = 1; w < 16; ++w) t += red[w][lane];
    if (beta != 0.0f) t = __builtin_fmaf(beta, ld_elem<DW_BF16>(dw, c), t);
    st_elem<DW_BF16>(dw, c, t);
  }
}

// ---- weight folding ------------------------------------------------------------
// W'[k, n] = weight[k] * W[k, n] (fp32 product, stored in W's dtype, bf16 rounded to
// nearest even): the RMSNorm weight moved into the rows of the next GEMM's B operand,
// so that rmsnorm(x) W = diag(1/rms) x W'.  VEC: 8 (bf16) or 4 (fp32) columns per
// thread with 16-byte accesses.
template <bool BF16, bool W_BF16, bool VEC>
__global__ void __launch_bounds__(256) norm_fold_weight_kernel(const void* w, const void* W, int64_t ldw,
                                                               int64_t K, int64_t N, void* out, int64_t ldo) {
  constexpr int EV = BF16 ? 8 : 4, ES = BF16 ? 2 : 4;
  const int64_t per_row = VEC ? N / EV : N;
  const int64_t n_items = K * per_row;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n_items; i += (int64_t)gridDim.x * 256) {
    const int64_t k = i / per_row, c = i - k * per_row;
    const float s = ld_elem<W_BF16>(w, (int)k);
    const char* src = (const char*)W + k * ldw * ES;
    char* dst = (char*)out + k * ldo * ES;
    if constexpr (VEC) {
      float v[EV];
      load_act<BF16>(src, (int)(c * EV), v);
#pragma unroll
      for (int e = 0; e < EV; ++e) v[e] *= s;
      store_act<BF16>(dst, (int)(c * EV), v);
    } else {
      st_elem<BF16>(dst, (int)c, ld_elem<BF16>(src, (int)c) * s);
    }
  }
}

int vec_per_lane(int dims, bool bf16) {
  const int per = (dims / (bf16 ? 8 : 4) + 63) / 64;
  return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;
}

template <bool BF16, bool W_BF16>
hipError_t fwd_one(const NormParams& p, bool vector_path, hipStream_t st) {
  if (!vector_path) {
    hipLaunchKernelGGL((norm_fwd_gen<BF16, W_BF16>), dim3((unsigned)p.rows), dim3(256), 0, st, p);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)((p.rows + 3) / 4)), block(256);
  switch (vec_per_lane(p.dims, BF16)) {
    case 1: hipLaunchKernelGGL((norm_fwd_vec<BF16, W_BF16, 1>), grid, block, 0, st, p); break;
    case 2: hipLaunchKernelGGL((norm_fwd_vec<BF16, W_BF16, 2>), grid, block, 0, st, p); break;
    case 4: hipLaunchKernelGGL((norm_fwd_vec<BF16, W_BF16, 4>), grid, block, 0, st, p); break;
    default: hipLaunchKernelGGL((norm_fwd_vec<BF16, W_BF16, 8>), grid, block, 0, st, p); break;
  }
  return hipGetLastError();
}

template <bool BF16, bool W_BF16>
hipError_t bwd_one(const NormParams& p, bool vector_path, hipStream_t st) {
  const int G = norm_bwd_grid(p.rows);
  if (!vector_path) {
    hipLaunchKernelGGL((norm_bwd_gen<BF16, W_BF16>), dim3((unsigned)G), dim3(256), 0, st, p);
  } else {
    const dim3 grid((unsigned)G), block(256);
    const size_t lds = p.dw ? (size_t)p.dims * sizeof(float) : 0;
    const int nv = vec_per_lane(p.dims, BF16);
    const bool full = p.dims == nv * 64 * (BF16 ? 8 : 4);  // every lane owns nv whole vectors
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, block, lds, st, p); };
    switch (nv) {
      case 1: full ? go(norm_bwd_vec<BF16, W_BF16, 1, true>) : go(norm_bwd_vec<BF16, W_BF16, 1, false>); break;
      case 2: full ? go(norm_bwd_vec<BF16, W_BF16, 2, true>) : go(norm_bwd_vec<BF16, W_BF16, 2, false>); break;
      case 4: full ? go(norm_bwd_vec<BF16, W_BF16, 4, true>) : go(norm_bwd_vec<BF16, W_BF16, 4, false>); break;
      default: full ? go(norm_bwd_vec<BF16, W_BF16, 8, true>) : go(norm_bwd_vec<BF16, W_BF16, 8, false>); break;
    }
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_norm_fwd(const NormParams& p, bool bf16, bool w_bf16, bool vector_path,
                           hipStream_t stream) {
  if (bf16) return w_bf16 ? fwd_one<true, true>(p, vector_path, stream)
                          : fwd_one<true, false>(p, vector_path, stream);
  return w_bf16 ? fwd_one<false, true>(p, vector_path, stream)
                : fwd_one<false, false>(p, vector_path, stream);
}

hipError_t launch_norm_fold_weight(const void* w, bool w_bf16, const void* W, int64_t ldw, int64_t K,
                                   int64_t N, bool bf16, void* out, int64_t ldo, bool vec, int cus,
                                   hipStream_t stream) {
  const int64_t items = K * (vec ? N / (bf16 ? 8 : 4) : N);
  const int64_t grid = std::min<int64_t>((items + 255) / 256, 8 * (int64_t)(cus > 0 ? cus : 256));
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), 0, stream, w, W, ldw, K, N, out, ldo);
  };
  if (bf16) {
    if (w_bf16) vec ? go(norm_fold_weight_kernel<true, true, true>) : go(norm_fold_weight_kernel<true, true, false>);
    else vec ? go(norm_fold_weight_kernel<true, false, true>) : go(norm_fold_weight_kernel<true, false, false>);
  } else {
    if (w_bf16) vec ? go(norm_fold_weight_kernel<false, true, true>) : go(norm_fold_weight_kernel<false, true, false>);
    else vec ? go(norm_fold_weight_kernel<false, false, true>) : go(norm_fold_weight_kernel<false, false, false>);
  }
  return hipGetLastError();
}

hipError_t launch_norm_bwd(const NormParams& p, bool bf16, bool w_bf16, bool dw_bf16,
                           bool vector_path, hipStream_t stream) {
  hipError_t e = bf16 ? (w_bf16 ? bwd_one<true, true>(p, vector_path, stream)
                                : bwd_one<true, false>(p, vector_path, stream))
                      : (w_bf16 ? bwd_one<false, true>(p, vector_path, stream)
                                : bwd_one<false, false>(p, vector_path, stream));
  if (e != hipSuccess || !p.dw) return e;
  const dim3 grid((unsigned)((p.dims + 63) / 64)), block(1024);
  const int G = norm_bwd_grid(p.rows);
  if (dw_bf16)
    hipLaunchKernelGGL(norm_dw_reduce<true>, grid, block, 0, stream, p.ws, G, p.dims, p.dw_beta, p.dw);
  else
    hipLaunchKernelGGL(norm_dw_reduce<false>, grid, block, 0, stream, p.ws, G, p.dims, p.dw_beta, p.dw);
  return hipGetLastError();
}

}  // namespace mig
