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
// element, so both the row-wise writes and the column-wise reads of the tile are
// conflict-free); global reads run along the source rows and global writes along
// the destination rows, both coalesced.
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

// One 64 x 64 tile per workgroup of 256 threads: each thread moves 16 elements.
__global__ void __launch_bounds__(256) convert_transpose_kernel(ConvParams p) {
  __shared__ float tile[CT][CT + 1];
  const int64_t r0 = (int64_t)blockIdx.y * CT, c0 = (int64_t)blockIdx.x * CT;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < CT / 4; ++k) {
    const int lr = ty + 4 * k;
    const int64_t r = r0 + lr, c = c0 + tx;
    if (r < p.rows && c < p.cols)
      tile[lr][tx] = load_any(p.src, (p.row0 + r) * p.src_ld + c, p.src_dtype);
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < CT / 4; ++k) {
    const int lc = ty + 4 * k;
    const int64_t c = c0 + lc, r = r0 + tx;  // dst row c, column r
    if (r < p.rows && c < p.cols) store_any(p.dst, c * p.dst_ld + r, p.dst_dtype, tile[tx][lc]);
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
  if (transpose) {
    const dim3 grid((unsigned)((p.cols + CT - 1) / CT), (unsigned)((p.rows + CT - 1) / CT));
    hipLaunchKernelGGL(convert_transpose_kernel, grid, dim3(256), 0, stream, p);
  } else {
    const int64_t n = p.rows * p.cols;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, (int64_t)cus * 16);
    hipLaunchKernelGGL(convert_copy_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace mig
