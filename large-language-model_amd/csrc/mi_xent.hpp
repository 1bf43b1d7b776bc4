// mi_xent.hpp -- launch interface of the softmax cross-entropy kernels
// (mi_xent.hip), called by the C ABI in mi_gemm.hip after it has validated the
// arguments.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mig {

struct XentParams {
  const void* logits;       // [rows, ld] bf16 or fp32
  const uint32_t* targets;  // [rows] class index per row
  float* row_loss;          // [rows] -log(max(p_target, 1e-15))
  void* grad;               // [rows, ldg] bf16 or fp32, or null (loss only)
  int64_t ld, ldg;          // leading dimensions in elements
  int rows, vocab;
  float scale;              // grad = scale * (softmax - onehot)
};

// Rows of at most this many 16-byte vectors are held in registers (one read of
// HBM per element); longer rows, or rows that are not whole 16-byte vectors,
// take the two-pass streaming kernel.
constexpr int XENT_THREADS = 512;
constexpr int XENT_MAX_VEC_PER_THREAD = 16;

hipError_t launch_xent(const XentParams& p, bool in_bf16, bool out_bf16, bool vector_path,
                       hipStream_t stream);

// loss_out[0] = scale * sum(row_loss[0 .. rows)), summed in a fixed order.
hipError_t launch_xent_mean(const float* row_loss, int rows, float scale, float* loss_out,
                            hipStream_t stream);

}  // namespace mig
