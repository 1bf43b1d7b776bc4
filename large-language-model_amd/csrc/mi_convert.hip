// mi_convert.hip -- weight layout and dtype conversion on the device, for loading
// checkpoints (gfx950).
//
// Reference: the checkpoint loader of the engine (cpp/src/Checkpoint.cpp:28-75,
// 407-535): bf16 and f16 file data widened to fp32 (bf16_to_f32, f16_to_f32), the
// [out, in] matrices of a Python/MLX file transposed to the engine's [in, out]
// (transpose_matrix), and the fused wqkv / w12 matrices cut into row ranges before
// the transpose (load_python_fused_tensor).  Here the file's bytes are copied to the
// device once and one kernel per destination does slice + transpose + conversion:
//   dst[r][c] = src[row0 + r][c]                      (transpose = 0)
//   dst[c][r] = src[row0 + r][c]                      (transpose = 1)
// for r < rows, c < cols, converted from the source dtype (fp32, bf16, f16) to the
// destination dtype (fp32, or bf16 rounded to nearest even).  bf16 -> fp32 and
// f16 -> fp32 are exact, as in the reference.
//
// HBM-bound.  The transpose goes through an LDS tile of 64 source rows x 256 source
// columns (rows padded by one element); global reads run along the source rows and
// global writes along the destination rows, 8 elements (16 bytes of bf16) per thread
// and run where aligned, with all of a thread's reads in flight before the tile is
// written to LDS.  The row-preserving copy moves 8 elements per thread where aligned.
// mi_convert_matrices puts many conversions into one launch of such tiles.  bf16 ->
// bf16 moves the bits as they are (NaN payloads included).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "mi_convert.hpp"
#include "mi_gemm_device.hpp"

namespace mig {
namespace {

__device__ __forceinline__ float load_any(const void* p, int64_t i, int dt) {
  if (dt == 1) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  if (dt == 2) return (float)((const _Float16*)p)[i];
  return ((const float*)p)[i];
}

__device__ __forceinline__ void store_any(void* p, int64_t i, int dt, float v) {
  if (dt == 1) ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16_rne(v);
  else ((float*)p)[i] = v;
}

// bf16 of a float that holds a bf16 value exactly: its upper half (== round to nearest
// even for such a value, and a NaN keeps its payload).
__device__ __forceinline__ uint32_t bf16_upper(float v) { return __float_as_uint(v) >> 16; }
__device__ __forceinline__ uint32_t pack_upper2(float lo, float hi) {
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}

constexpr int TR = 64, TC = 256;  // transpose / batch tile: source rows x source columns

template <int DT>
__device__ __forceinline__ float ld1(const void* p, int64_t i) {
  if constexpr (DT == 1) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  else if constexpr (DT == 2) return (float)((const _Float16*)p)[i];
  else return ((const float*)p)[i];
}

// Four consecutive elements at element index i (i % 4 == 0, base aligned).
template <int DT>
__device__ __forceinline__ void ld4(const void* p, int64_t i, float* v) {
  if constexpr (DT == 0) {
    const float4 q = *(const float4*)((const float*)p + i);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else {
    const uint2 q = *(const uint2*)((const uint16_t*)p + i);
    if constexpr (DT == 1) {
      v[0] = __uint_as_float(q.x << 16); v[1] = __uint_as_float(q.x & 0xffff0000u);
      v[2] = __uint_as_float(q.y << 16); v[3] = __uint_as_float(q.y & 0xffff0000u);
    } else {
      const _Float16* h = (const _Float16*)&q;
      v[0] = (float)h[0]; v[1] = (float)h[1]; v[2] = (float)h[2]; v[3] = (float)h[3];
    }
  }
}

// Eight consecutive elements at element index i (i % 8 == 0, base aligned).
template <int DT>
__device__ __forceinline__ void ld8(const void* p, int64_t i, float* v) {
  if constexpr (DT == 0) {
    ld4<0>(p, i, v);
    ld4<0>(p, i + 4, v + 4);
  } else {
    const uint4 q = *(const uint4*)((const uint16_t*)p + i);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == 1) {
        v[2 * j] = __uint_as_float(w[j] << 16);
        v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
      } else {
        const _Float16* h = (const _Float16*)&w[j];
        v[2 * j] = (float)h[0];
        v[2 * j + 1] = (float)h[1];
      }
    }
  }
}

// Stores: RAW (source bf16, destination bf16) takes the upper halves, anything else
// rounds to nearest even.
template <int DT, bool RAW>
__device__ __forceinline__ void st1(void* p, int64_t i, float v) {
  if constexpr (DT == 1) ((uint16_t*)p)[i] = (uint16_t)(RAW ? bf16_upper(v) : f32_to_bf16_rne(v));
  else ((float*)p)[i] = v;
}

template <bool RAW>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return RAW ? pack_upper2(lo, hi) : pack_bf16x2(lo, hi);
}

template <int DT, bool RAW>
__device__ __forceinline__ void st4(void* p, int64_t i, const float* v) {
  if constexpr (DT == 1) *(uint2*)((uint16_t*)p + i) = make_uint2(pack2<RAW>(v[0], v[1]), pack2<RAW>(v[2], v[3]));
  else *(float4*)((float*)p + i) = make_float4(v[0], v[1], v[2], v[3]);
}

template <int DT, bool RAW>
__device__ __forceinline__ void st8(void* p, int64_t i, const float* v) {
  if constexpr (DT == 1) {
    *(uint4*)((uint16_t*)p + i) = make_uint4(pack2<RAW>(v[0], v[1]), pack2<RAW>(v[2], v[3]),
                                             pack2<RAW>(v[4], v[5]), pack2<RAW>(v[6], v[7]));
  } else {
    st4<0, RAW>(p, i, v);
    st4<0, RAW>(p, i + 4, v + 4);
  }
}

// 8 consecutive elements at element index i: vec 2 one access per 8 (16 bytes of
// bf16 / f16), vec 1 two 4-element accesses.
template <int DT>
__device__ __forceinline__ void ld_run(const void* p, int64_t i, float* v, int vec) {
  if (vec == 2) {
    ld8<DT>(p, i, v);
  } else {
    ld4<DT>(p, i, v);
    ld4<DT>(p, i + 4, v + 4);
  }
}

template <int DT, bool RAW>
__device__ __forceinline__ void st_run(void* p, int64_t i, const float* v, int vec) {
  if (vec == 2) {
    st8<DT, RAW>(p, i, v);
  } else {
    st4<DT, RAW>(p, i, v);
    st4<DT, RAW>(p, i + 4, v + 4);
  }
}

// One tile of TR source rows x TC source columns per workgroup of 256 threads.
// Reads: 32 threads per 256-element source row, 8 consecutive elements each, 8 rows
// per pass, 8 passes (512-byte row segments of bf16: longer source segments beat
// longer destination segments when the data does not fit the last-level cache);
// writes: 8 threads per 64-element destination row, 8 elements each, 32 rows per
// pass.  vec (uniform): 2 or 1 when every run is aligned for 8- or 4-element
// accesses, 0 for single elements.  An interior tile issues all eight reads before
// any LDS write and all eight LDS reads before any global write; edge tiles take
// single elements under bounds checks.  LDS row lr, column j sits at bank
// (lr + j) % 64, so the reads down a column (8 runs of 8 rows, 8 columns per wave)
// touch 64 distinct banks per element step.
template <int SRC, int DST>
__device__ __forceinline__ void transpose_tile(const ConvParams& p, int vec, int64_t r0, int64_t c0,
                                               float (*tile)[TC + 1]) {
  constexpr bool RAW = SRC == 1 && DST == 1;
  const int t = threadIdx.x, rj = (t & 31) * 8, rs = t >> 5, wj = (t & 7) * 8, ws = t >> 3;
  const bool fast = vec && c0 + TC <= p.cols && r0 + TR <= p.rows;
  float v[8][8];
  if (fast) {
#pragma unroll
    for (int k = 0; k < 8; ++k) ld_run<SRC>(p.src, (p.row0 + r0 + rs + 8 * k) * p.src_ld + c0 + rj, v[k], vec);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t r = r0 + rs + 8 * k, base = (p.row0 + r) * p.src_ld + c0 + rj;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        v[k][e] = r < p.rows && c0 + rj + e < p.cols ? ld1<SRC>(p.src, base + e) : 0.0f;
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[rs + 8 * k][rj + e] = v[k][e];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) v[k][e] = tile[wj + e][ws + 32 * k];
  if (fast) {
#pragma unroll
    for (int k = 0; k < 8; ++k) st_run<DST, RAW>(p.dst, (c0 + ws + 32 * k) * p.dst_ld + r0 + wj, v[k], vec);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t c = c0 + ws + 32 * k;  // destination row
      if (c >= p.cols) continue;
      const int64_t base = c * p.dst_ld + r0 + wj;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (r0 + wj + e < p.rows) st1<DST, RAW>(p.dst, base + e, v[k][e]);
    }
  }
}

// The same tile copied without the transpose (global to global, the read runs).
template <int SRC, int DST>
__device__ __forceinline__ void copy_tile(const ConvParams& p, int vec, int64_t r0, int64_t c0) {
  constexpr bool RAW = SRC == 1 && DST == 1;
  const int t = threadIdx.x, rj = (t & 31) * 8, rs = t >> 5;
  if (vec && c0 + TC <= p.cols && r0 + TR <= p.rows) {
    float v[8][8];
#pragma unroll
    for (int k = 0; k < 8; ++k) ld_run<SRC>(p.src, (p.row0 + r0 + rs + 8 * k) * p.src_ld + c0 + rj, v[k], vec);
#pragma unroll
    for (int k = 0; k < 8; ++k) st_run<DST, RAW>(p.dst, (r0 + rs + 8 * k) * p.dst_ld + c0 + rj, v[k], vec);
    return;
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int64_t r = r0 + rs + 8 * k;
    if (r >= p.rows) continue;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t c = c0 + rj + e;
      if (c < p.cols) st1<DST, RAW>(p.dst, r * p.dst_ld + c, ld1<SRC>(p.src, (p.row0 + r) * p.src_ld + c));
    }
  }
}

template <int SRC, int DST>
__global__ void __launch_bounds__(256) convert_transpose_kernel(ConvParams p, int vec) {
  __shared__ float tile[TR][TC + 1];
  transpose_tile<SRC, DST>(p, vec, (int64_t)blockIdx.y * TR, (int64_t)blockIdx.x * TC, tile);
}

// A launch of several conversions: job j owns the tiles [tile0, tile0 + its tile
// count) of a 1-D grid, row-major over its tiles_x columns of tiles.  The job table
// travels in the kernel arguments; the workgroup picks its job with uniform selects
// over the fixed-size table (no indexed access to the argument block).
struct ConvBatchJob {
  ConvParams p;
  int64_t tile0, tiles_x;
  int32_t transpose, vec;
};

struct ConvBatch {
  ConvBatchJob job[CONV_BATCH];
  int32_t n;
};

template <int SRC, int DST>
__global__ void __launch_bounds__(256) convert_batch_kernel(ConvBatch b) {
  __shared__ float tile[TR][TC + 1];
  const int64_t bid = blockIdx.x;
  int j = 0;
#pragma unroll
  for (int i = 1; i < CONV_BATCH; ++i)
    if (i < b.n && bid >= b.job[i].tile0) j = i;
  ConvBatchJob J = b.job[0];
#pragma unroll
  for (int i = 1; i < CONV_BATCH; ++i)
    if (i == j) J = b.job[i];
  const int64_t t = bid - J.tile0, r0 = t / J.tiles_x * TR, c0 = t % J.tiles_x * TC;
  if (J.transpose) transpose_tile<SRC, DST>(J.p, J.vec, r0, c0, tile);
  else copy_tile<SRC, DST>(J.p, J.vec, r0, c0);
}

// Row-preserving copy, VE (4 or 8) elements per thread and access each way: x covers
// the columns, y the rows (strided past 65535).  Needs cols, both leading dimensions
// and the source row offset to be multiples of VE and both bases aligned to VE
// elements.
template <int SRC, int DST, int VE>
__global__ void __launch_bounds__(256) convert_copy_vec_kernel(ConvParams p) {
  constexpr bool RAW = SRC == 1 && DST == 1;
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * VE;
  if (c >= p.cols) return;
  for (int64_t r = blockIdx.y; r < p.rows; r += gridDim.y) {
    float v[VE];
    if constexpr (VE == 8) {
      ld8<SRC>(p.src, (p.row0 + r) * p.src_ld + c, v);
      st8<DST, RAW>(p.dst, r * p.dst_ld + c, v);
    } else {
      ld4<SRC>(p.src, (p.row0 + r) * p.src_ld + c, v);
      st4<DST, RAW>(p.dst, r * p.dst_ld + c, v);
    }
  }
}

__global__ void __launch_bounds__(256) convert_copy_kernel(ConvParams p) {
  const int64_t n = p.rows * p.cols;
  const bool raw = p.src_dtype == 1 && p.dst_dtype == 1;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / p.cols, c = i - r * p.cols;
    if (raw) {
      ((uint16_t*)p.dst)[r * p.dst_ld + c] = ((const uint16_t*)p.src)[(p.row0 + r) * p.src_ld + c];
    } else {
      store_any(p.dst, r * p.dst_ld + c, p.dst_dtype,
                load_any(p.src, (p.row0 + r) * p.src_ld + c, p.src_dtype));
    }
  }
}

// rows x cols bf16 -> rows x dst_cols bf16 (dst_cols >= cols, both multiples of 8), the
// columns past cols written as zeros: one thread per 8-element chunk of a destination
// row; VEC: 16-byte source loads (source base and row pitch 16-byte aligned).
template <bool VEC>
__global__ void __launch_bounds__(256) pad_rows_kernel(const uint16_t* src, int64_t src_ld, int64_t rows,
                                                       int64_t cols, uint16_t* dst, int64_t dst_cols) {
  const int64_t cpr = dst_cols / 8;
  const int64_t n = rows * cpr;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / cpr, c = (i - r * cpr) * 8;
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (c < cols) {
      const uint16_t* s = src + r * src_ld + c;
      if constexpr (VEC) {
        v = *(const u32x4_t*)s;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (uint32_t)s[2 * e] | ((uint32_t)s[2 * e + 1] << 16);
      }
    }
    *(u32x4_t*)(dst + r * dst_cols + c) = v;
  }
}

}  // namespace

hipError_t launch_pad_rows(const void* src, int64_t src_ld, int64_t rows, int64_t cols, void* dst,
                           int64_t dst_cols, int cus, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  if (cols % 8 || dst_cols % 8 || cols > dst_cols || src_ld < cols || ((uintptr_t)dst & 15u))
    return hipErrorInvalidValue;
  const int64_t n = rows * (dst_cols / 8);
  const int64_t grid = std::min<int64_t>((n + 255) / 256, 8 * (int64_t)(cus > 0 ? cus : 256));
  const bool vec = ((uintptr_t)src & 15u) == 0 && src_ld % 8 == 0;
  if (vec)
    hipLaunchKernelGGL(pad_rows_kernel<true>, dim3((unsigned)grid), dim3(256), 0, stream, (const uint16_t*)src,
                       src_ld, rows, cols, (uint16_t*)dst, dst_cols);
  else
    hipLaunchKernelGGL(pad_rows_kernel<false>, dim3((unsigned)grid), dim3(256), 0, stream,
                       (const uint16_t*)src, src_ld, rows, cols, (uint16_t*)dst, dst_cols);
  return hipGetLastError();
}

hipError_t launch_convert(const ConvParams& p, bool transpose, int cus, hipStream_t stream) {
  const int ses = p.src_dtype == 0 ? 4 : 2, des = p.dst_dtype == 0 ? 4 : 2;
  auto aligned = [&](int n) {
    return p.src_ld % n == 0 && p.dst_ld % n == 0 && (p.row0 * p.src_ld) % n == 0 &&
           (uintptr_t)p.src % (n * ses) == 0 && (uintptr_t)p.dst % (n * des) == 0;
  };
  const int vec = aligned(4);
  if (!transpose && vec && p.cols % 4 == 0) {
    const int ve = aligned(8) && p.cols % 8 == 0 ? 8 : 4;
    const dim3 grid((unsigned)((p.cols + 256 * ve - 1) / (256 * ve)), (unsigned)std::min<int64_t>(p.rows, 65535));
    auto go = [&](auto k8, auto k4) {
      if (ve == 8) hipLaunchKernelGGL(k8, grid, dim3(256), 0, stream, p);
      else hipLaunchKernelGGL(k4, grid, dim3(256), 0, stream, p);
    };
    if (p.dst_dtype == 1) {
      if (p.src_dtype == 1) go(convert_copy_vec_kernel<1, 1, 8>, convert_copy_vec_kernel<1, 1, 4>);
      else if (p.src_dtype == 2) go(convert_copy_vec_kernel<2, 1, 8>, convert_copy_vec_kernel<2, 1, 4>);
      else go(convert_copy_vec_kernel<0, 1, 8>, convert_copy_vec_kernel<0, 1, 4>);
    } else {
      if (p.src_dtype == 1) go(convert_copy_vec_kernel<1, 0, 8>, convert_copy_vec_kernel<1, 0, 4>);
      else if (p.src_dtype == 2) go(convert_copy_vec_kernel<2, 0, 8>, convert_copy_vec_kernel<2, 0, 4>);
      else go(convert_copy_vec_kernel<0, 0, 8>, convert_copy_vec_kernel<0, 0, 4>);
    }
    return hipGetLastError();
  }
  if (transpose) {
    const dim3 grid((unsigned)((p.cols + TC - 1) / TC), (unsigned)((p.rows + TR - 1) / TR));
    const int v = aligned(8) ? 2 : vec;
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, p, v); };
    if (p.dst_dtype == 1) {
      if (p.src_dtype == 1) go(convert_transpose_kernel<1, 1>);
      else if (p.src_dtype == 2) go(convert_transpose_kernel<2, 1>);
      else go(convert_transpose_kernel<0, 1>);
    } else {
      if (p.src_dtype == 1) go(convert_transpose_kernel<1, 0>);
      else if (p.src_dtype == 2) go(convert_transpose_kernel<2, 0>);
      else go(convert_transpose_kernel<0, 0>);
    }
  } else {
    const int64_t n = p.rows * p.cols;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, (int64_t)cus * 16);
    hipLaunchKernelGGL(convert_copy_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p);
  }
  return hipGetLastError();
}

namespace {

// 2 when every 8-element run of p is aligned for one access per 8 elements, 1 for 4,
// 0 otherwise.
int vec_ok(const ConvParams& p) {
  const int ses = p.src_dtype == 0 ? 4 : 2, des = p.dst_dtype == 0 ? 4 : 2;
  auto aligned = [&](int n) {
    return p.src_ld % n == 0 && p.dst_ld % n == 0 && (p.row0 * p.src_ld) % n == 0 &&
           (uintptr_t)p.src % (n * ses) == 0 && (uintptr_t)p.dst % (n * des) == 0;
  };
  return aligned(8) ? 2 : aligned(4) ? 1 : 0;
}

template <int SRC, int DST>
hipError_t launch_batch_group(const ConvParams* jobs, const int* transpose, const int64_t* idx,
                              int64_t n, hipStream_t stream) {
  ConvBatch b;
  int64_t i = 0;
  while (i < n) {
    b.n = 0;
    int64_t tiles = 0;
    // at most CONV_BATCH jobs and 2^31 - 1 tiles per launch (each job has fewer than 2^30)
    while (i < n && b.n < CONV_BATCH) {
      const ConvParams& p = jobs[idx[i]];
      const int64_t tx = (p.cols + TC - 1) / TC, ty = (p.rows + TR - 1) / TR;
      if (b.n > 0 && tiles + tx * ty > INT32_MAX) break;
      ConvBatchJob& J = b.job[b.n++];
      J.p = p;
      J.tile0 = tiles;
      J.tiles_x = tx;
      J.transpose = transpose[idx[i]] ? 1 : 0;
      J.vec = vec_ok(p);
      tiles += tx * ty;
      ++i;
    }
    for (int k = b.n; k < CONV_BATCH; ++k) b.job[k] = b.job[0];
    hipLaunchKernelGGL((convert_batch_kernel<SRC, DST>), dim3((unsigned)tiles), dim3(256), 0, stream, b);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_convert_batch(const ConvParams* jobs, const int* transpose, int64_t n,
                                hipStream_t stream) {
  std::vector<int64_t> idx;
  idx.reserve((size_t)n);
  for (int sd = 0; sd < 3; ++sd) {
    for (int dd = 0; dd < 2; ++dd) {
      idx.clear();
      for (int64_t i = 0; i < n; ++i)
        if (jobs[i].src_dtype == sd && jobs[i].dst_dtype == dd && jobs[i].rows > 0 && jobs[i].cols > 0)
          idx.push_back(i);
      if (idx.empty()) continue;
      const int64_t m = (int64_t)idx.size();
      hipError_t e;
      if (dd == 1) {
        e = sd == 1 ? launch_batch_group<1, 1>(jobs, transpose, idx.data(), m, stream)
            : sd == 2 ? launch_batch_group<2, 1>(jobs, transpose, idx.data(), m, stream)
                      : launch_batch_group<0, 1>(jobs, transpose, idx.data(), m, stream);
      } else {
        e = sd == 1 ? launch_batch_group<1, 0>(jobs, transpose, idx.data(), m, stream)
            : sd == 2 ? launch_batch_group<2, 0>(jobs, transpose, idx.data(), m, stream)
                      : launch_batch_group<0, 0>(jobs, transpose, idx.data(), m, stream);
      }
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

}  // namespace mig
