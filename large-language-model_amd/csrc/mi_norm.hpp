// mi_norm.hpp -- launch interface of the RMSNorm kernels (mi_norm.hip), called
// by the C ABI in mi_gemm.hip after it has validated the arguments.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mig {

struct NormParams {
  void* x;            // [rows, ld] input; forward with r: updated in place to x + r
  const void* r;      // forward: residual added into x first; backward: gradient added to dx
  const void* w;      // [dims] weight
  void* y;            // forward output [rows, ld], or null: rstd only
  const void* dy;     // backward: gradient of y [rows, ld]
  void* dx;           // backward output [rows, ld]
  float* rstd;        // forward: optional [rows] 1 / rms
  void* dw;           // backward: optional [dims] weight gradient
  float* ws;          // backward with dw: [norm_bwd_grid(rows), dims] partial sums
  int64_t ld;         // leading dimension of every row array (elements)
  int rows, dims;
  float eps, dw_beta;
};

// Workgroups of the backward kernels (each owns one row of the dw workspace).
inline int norm_bwd_grid(int rows) {
  const int g = (rows + 3) / 4;
  return g < 512 ? (g < 1 ? 1 : g) : 512;
}

// Rows of at most this many 16-byte vectors per lane (64 lanes) take the
// register kernels: 4096 bf16 or 2048 fp32 values.
constexpr int NORM_MAX_VEC_PER_LANE = 8;

hipError_t launch_norm_fwd(const NormParams& p, bool bf16, bool w_bf16, bool vector_path,
                           hipStream_t stream);
hipError_t launch_norm_bwd(const NormParams& p, bool bf16, bool w_bf16, bool dw_bf16,
                           bool vector_path, hipStream_t stream);
// out[k, n] = w[k] * W[k, n] for k < K, n < N (W's dtype; vec: 16-byte column groups).
hipError_t launch_norm_fold_weight(const void* w, bool w_bf16, const void* W, int64_t ldw, int64_t K,
                                   int64_t N, bool bf16, void* out, int64_t ldo, bool vec, int cus,
                                   hipStream_t stream);

}  // namespace mig
