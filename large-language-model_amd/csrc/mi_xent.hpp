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

// Vocabulary chunks (bf16 logits of columns [c0, c0 + n) in L[rows][ldl]): pass 1
// merges each chunk into the running (run_m, run_s) and records the target's logit in
// xy; finish writes the row losses and turns run_s into scale / s; pass 2 overwrites a
// recomputed chunk with its gradient.
hipError_t launch_xent_chunk_stats(const void* L, int64_t ldl, int rows, int n, int c0,
                                   const uint32_t* targets, float* run_m, float* run_s, float* xy, bool first,
                                   hipStream_t stream);
hipError_t launch_xent_chunk_finish(int rows, int vocab, const uint32_t* targets, const float* run_m,
                                    float* run_s, const float* xy, float scale, float* row_loss,
                                    hipStream_t stream);
hipError_t launch_xent_chunk_grad(void* L, int64_t ldl, int rows, int n, int c0, const uint32_t* targets,
                                  const float* run_m, const float* run_inv, float scale, hipStream_t stream);

}  // namespace mig
