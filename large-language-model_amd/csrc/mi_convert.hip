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
// HBM-bound.  The transpose goes through a 64 x 64 LDS tile (rows padded by one
// element); global reads run along the source rows and global writes along the
// destination rows, 4 elements (8 or 16 bytes) per access where aligned.
#include <hip/hip_runtime.h>

#include <algorithm>

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

constexpr int CT = 64;  // tile edge

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

template <int DT>
__device__ __forceinline__ void st1(void* p, int64_t i, float v) {
  if constexpr (DT == 1) ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16_rne(v);
  else ((float*)p)[i] = v;
}

template <int DT>
__device__ __forceinline__ void st4(void* p, int64_t i, const float* v) {
  if constexpr (DT == 1) *(uint2*)((uint16_t*)p + i) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
  else *(float4*)((float*)p + i) = make_float4(v[0], v[1], v[2], v[3]);
}

// One 64 x 64 tile per workgroup of 256 threads.  Reads: each thread takes 4 runs of
// 4 consecutive source elements (16 threads per 64-element source row); writes: 4
// runs of 4 consecutive destination elements.  vec (uniform) says every run is
// aligned for one 8- or 16-byte access; edge tiles fall back to single elements.
template <int SRC, int DST>
__global__ void __launch_bounds__(256) convert_transpose_kernel(ConvParams p, int vec) {
  __shared__ float tile[CT][CT + 1];
  const int64_t r0 = (int64_t)blockIdx.y * CT, c0 = (int64_t)blockIdx.x * CT;
  const int t = threadIdx.x, j4 = (t & 15) * 4, sub = t >> 4;
  const bool full_c = c0 + CT <= p.cols, full_r = r0 + CT <= p.rows;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int lr = sub + 16 * k;
    const int64_t r = r0 + lr;
    if (r >= p.rows) continue;
    const int64_t base = (p.row0 + r) * p.src_ld + c0 + j4;
    float v[4];
    if (vec && full_c) {
      ld4<SRC>(p.src, base, v);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = c0 + j4 + e < p.cols ? ld1<SRC>(p.src, base + e) : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[lr][j4 + e] = v[e];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int lc = sub + 16 * k;
    const int64_t c = c0 + lc;  // destination row
    if (c >= p.cols) continue;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = tile[j4 + e][lc];
    const int64_t base = c * p.dst_ld + r0 + j4;
    if (vec && full_r) {
      st4<DST>(p.dst, base, v);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (r0 + j4 + e < p.rows) st1<DST>(p.dst, base + e, v[e]);
    }
  }
}

// Row-preserving copy, 4 elements (one 8- or 16-byte access each way) per thread: x
// covers the columns, y the rows (strided past 65535).  Needs the alignment of the
// transpose's vector path.
template <int SRC, int DST>
__global__ void __launch_bounds__(256) convert_copy_vec_kernel(ConvParams p) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= p.cols) return;
  for (int64_t r = blockIdx.y; r < p.rows; r += gridDim.y) {
    float v[4];
    ld4<SRC>(p.src, (p.row0 + r) * p.src_ld + c, v);
    st4<DST>(p.dst, r * p.dst_ld + c, v);
  }
}

__global__ void __launch_bounds__(256) convert_copy_kernel(ConvParams p) {
  const int64_t n = p.rows * p.cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / p.cols, c = i - r * p.cols;
    store_any(p.dst, r * p.dst_ld + c, p.dst_dtype,
              load_any(p.src, (p.row0 + r) * p.src_ld + c, p.src_dtype));
  }
}

}  // namespace

hipError_t launch_convert(const ConvParams& p, bool transpose, int cus, hipStream_t stream) {
  const int ses = p.src_dtype == 0 ? 4 : 2, des = p.dst_dtype == 0 ? 4 : 2;
  const int vec = p.src_ld % 4 == 0 && p.dst_ld % 4 == 0 && (p.row0 * p.src_ld) % 4 == 0 &&
                  (uintptr_t)p.src % (4 * ses) == 0 && (uintptr_t)p.dst % (4 * des) == 0;
  if (!transpose && vec && p.cols % 4 == 0) {
    const dim3 grid((unsigned)((p.cols + 1023) / 1024), (unsigned)std::min<int64_t>(p.rows, 65535));
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, p); };
    if (p.dst_dtype == 1) {
      if (p.src_dtype == 1) go(convert_copy_vec_kernel<1, 1>);
      else if (p.src_dtype == 2) go(convert_copy_vec_kernel<2, 1>);
      else go(convert_copy_vec_kernel<0, 1>);
    } else {
      if (p.src_dtype == 1) go(convert_copy_vec_kernel<1, 0>);
      else if (p.src_dtype == 2) go(convert_copy_vec_kernel<2, 0>);
      else go(convert_copy_vec_kernel<0, 0>);
    }
    return hipGetLastError();
  }
  if (transpose) {
    const dim3 grid((unsigned)((p.cols + CT - 1) / CT), (unsigned)((p.rows + CT - 1) / CT));
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, p, vec); };
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

}  // namespace mig
