// mi_attn.hpp -- launch interface of the fused attention kernels (mi_attn.hip),
// called by the C ABI in mi_gemm.hip after it has validated the arguments.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mig {

struct FaParams {
  const void* Q;  // [B, nH, T, d] bf16
  const void* K;  // [B, nKV, T, d] bf16
  const void* V;  // [B, nKV, T, d] bf16
  void* O;        // bf16: [B, nH, T, d], or [B, T, nH*d] when o_bthd
  float* lse;     // [B, nH, T] natural-log row log-sum-exp of the scaled scores, or null
  int B, nH, nKV, T, group;  // group = nH / nKV query heads per KV head
  int causal, o_bthd;
  int q_blocks;              // flash_fwd_blocks(T)
  float scale_log2;          // log2(e) / sqrt(d)
};

struct FbParams {
  const void* Q;   // [B, nH, T, d] bf16
  const void* K;   // [B, nKV, T, d] bf16
  const void* V;   // [B, nKV, T, d] bf16
  const void* O;   // forward output, layout as dO
  const void* dO;  // bf16: [B, nH, T, d], or [B, T, nH*d] when o_bthd
  const float* lse;  // [B, nH, T] from the forward
  void* dQ;        // [B, nH, T, d] bf16
  void* dK;        // [B, nKV, T, d] bf16
  void* dV;        // [B, nKV, T, d] bf16
  float* delta;    // [B, nH, T] workspace: rowsum(dO * O)
  void* dsT;       // null, or [B, nH, T, T] bf16 workspace receiving dS^T (key-major):
                   // then dQ is left to a batched GEMM dQ = scale * dS K by the caller
  int B, nH, nKV, T, group;
  int causal, o_bthd;
  int q_blocks;    // flash_fwd_blocks(T)
  int k_blocks;    // flash_bwd_key_blocks(T)
  float scale_log2;  // log2(e) / sqrt(d)
  float scale;       // 1 / sqrt(d)
};

// Query blocks per (batch, head) of the forward kernel.
int flash_fwd_blocks(int T);

// Key blocks per (batch, KV head) of the dK/dV kernel.
int flash_bwd_key_blocks(int T);

// Launch the backward kernels (head_dim 128) on `stream`: dQ and D, then dK / dV.
hipError_t launch_flash_bwd(const FbParams& p, int head_dim, hipStream_t stream);

// Launch the forward kernel (head_dim 128) on `stream`.
hipError_t launch_flash_fwd(const FaParams& p, int head_dim, hipStream_t stream);

}  // namespace mig
