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

// Limits of the balanced dK/dV schedule carried in the kernel arguments.
constexpr int FB_MAX_UNITS = 192;
constexpr int FB_MAX_SPLIT = 64;

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
  // Balanced dK/dV schedule (dS^T form, set by launch_flash_bwd).  The iterations of
  // a key block (its group heads x query tiles, head-major) are cut into units of
  // about equal length; a workgroup runs one unit of one (batch, KV head), largest
  // units first.  A key block cut into several units writes fp32 partial dK / dV,
  // summed in unit order by a reduction kernel.  n_units = 0: one workgroup per key
  // block, all its iterations, no partials.
  float* part;        // [B * nKV][n_slots][dK, dV][128 keys][d] fp32 partials
  size_t part_bytes;  // room at `part` (host side)
  int cus;            // compute units of the device (host side)
  int n_units, n_slots, n_split;
  uint32_t unit_kbi[FB_MAX_UNITS];    // key block | (partial slot + 1) << 16 (0: direct output)
  uint32_t unit_range[FB_MAX_UNITS];  // first iteration | end iteration << 16
  uint32_t split[FB_MAX_SPLIT];       // key block | first slot << 12 | units << 24
};

// Query blocks per (batch, head) of the forward kernel.
int flash_fwd_blocks(int T);

// Key blocks per (batch, KV head) of the dK/dV kernel.
int flash_bwd_key_blocks(int T);

// Bytes of fp32 dK / dV partials the balanced dK/dV schedule may need (dS^T form).
size_t flash_bwd_partial_bytes(int64_t B, int64_t nH, int64_t T);

// Launch the backward kernels (head_dim 64 or 128) on `stream`: dQ and D, then dK / dV
// (and, with a balanced schedule, the reduction of the partials).
hipError_t launch_flash_bwd(const FbParams& p, int head_dim, hipStream_t stream);

// Launch the forward kernel (head_dim 64 or 128) on `stream`.
hipError_t launch_flash_fwd(const FaParams& p, int head_dim, hipStream_t stream);

}  // namespace mig
