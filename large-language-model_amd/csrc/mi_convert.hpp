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

constexpr int CONV_BATCH = 16;  // jobs per launch of launch_convert_batch

hipError_t launch_convert(const ConvParams& p, bool transpose, int cus, hipStream_t stream);

// Several conversions in as few launches as possible: jobs of one (source, destination)
// dtype pair go into one launch of 64 x 256 tiles (CONV_BATCH jobs per launch at most).
// The caller has validated every job and checked that no destination overlaps another
// job's source or destination (the tiles of a launch run in any order).
hipError_t launch_convert_batch(const ConvParams* jobs, const int* transpose, int64_t n,
                                hipStream_t stream);

// Internal (the C++ bridge's padded attention operands): rows x cols bf16 from `src`
// (row pitch src_ld elements) into rows of dst_cols elements at `dst` (16-byte
// aligned), columns cols .. dst_cols-1 set to zero.  cols and dst_cols multiples of 8.
hipError_t launch_pad_rows(const void* src, int64_t src_ld, int64_t rows, int64_t cols, void* dst,
                           int64_t dst_cols, int cus, hipStream_t stream);

}  // namespace mig
