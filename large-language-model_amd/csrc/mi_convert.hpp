// mi_convert.hpp -- launch interface of the weight conversion kernels
// (mi_convert.hip), called by the C ABI in mi_gemm.hip after it has validated
// the arguments.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mig {

struct ConvParams {
  const void* src;
  void* dst;
  int64_t src_ld, dst_ld;    // elements
  int64_t row0, rows, cols;  // source rows [row0, row0 + rows), columns [0, cols)
  int src_dtype, dst_dtype;  // 0 fp32, 1 bf16, 2 f16 (source only)
};

hipError_t launch_convert(const ConvParams& p, bool transpose, int cus, hipStream_t stream);

}  // namespace mig
