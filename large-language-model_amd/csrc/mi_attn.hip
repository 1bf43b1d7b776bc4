// mi_attn.hip -- fused GQA flash-attention forward for gfx950 (bf16 in, fp32 softmax
// and accumulation, bf16 out).
//
// Replaces the reference's attention forward: Attention::forward (Attention.cpp:
// 236-280: kv_h = h / (nH/nKV), S = Q K^T / sqrt(d), causal k <= q, stable softmax,
// O = P V written to [B, T, nH*d]) and metal_bridge::flash_attn_fwd
// (MetalBridge.hpp:49-51, flash_attn_fwd.metal: online softmax, output
// [B, nH, T, d]).  S and P never leave the chip: one workgroup owns 128 query rows of
// one (batch, head), streams the 64-key K/V blocks of the shared KV head through a
// two-stage LDS ring and keeps the running max, running sum and the 128 x d output
// accumulator in registers (FlashAttention-2 style online softmax).
//
// Work split: 4 waves x 32 query rows, two workgroups per CU, so each SIMD holds
// two waves and one wave's softmax (VALU) runs under the other's MFMAs.  Per
// 64-key block a wave computes
//   S[32 q x 64 keys] = K Q^T  (first MFMA operand K, so each lane owns one query
//                               row and 32 of the block's keys for that row),
//   the online-softmax update on those registers, and
//   O[32 q x d] += P V         (first operand V^T via the transposing LDS read, second
//                               operand P straight from the S registers).
// The S registers of a lane hold keys 8q + 4h + e (h = lane / 32) of each 32-key
// half; reading the K rows in the order that swaps bits 2 and 3 of the key index
// makes those registers hold, in order, exactly the 8-key runs the P operand of
// v_mfma_f32_32x32x16_bf16 needs, so P never goes through LDS.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <functional>
#include <queue>
#include <vector>

#include "mi_attn.hpp"
#include "mi_gemm_dlds.hpp"

namespace mig {

namespace {

constexpr int FA_BQ = 128;   // query rows per workgroup (32 per wave)
constexpr int FA_BK = 64;    // keys per K/V block
constexpr float FA_TAU = 8.0f;  // growth of a row max (log2 units of p) that forces a rescale

// Workgroup b runs on XCD b mod 8, as the (b / 8)-th there.  The n work items come
// heaviest first in runs of g that should share one L2 (the query heads of a KV
// group); run r goes to XCD r mod 8, so every XCD gets the same mix of weights,
// heaviest first, and keeps whole runs.  (A contiguous range per XCD would give
// XCD 0 all of the heaviest items: with B * nH = 128 and 8 causal query blocks,
// XCD 0 would run every 16-block query block and XCD 7 every 2-block one.)  Items
// past the last whole round of 8g runs keep their index.
__device__ __forceinline__ int fa_xcd_spread(int bid, int n, int g) {
  const int round = 8 * g, nfull = n - n % round;
  if (bid >= nfull) return bid;
  const int x = bid % 8, j = bid / 8;
  return ((j / g) * 8 + x) * g + j % g;
}

// Key row read by lane row p (0..31) of a 32-key half: bits 2 and 3 swapped.
__device__ __forceinline__ int fa_key_perm(int p) {
  return (p & ~0xC) | ((p & 4) << 1) | ((p & 8) >> 1);
}

// LDS layout of a [row][d] bf16 tile of 64 rows (a K, V, Q or dO block): rows of
// ROW bytes in 16-byte chunks, the chunk position XOR-swizzled by the row.  Head
// dimension 128 (256-byte rows, 16 chunks, four rows per 1 KB DMA block) and 64
// (128-byte rows, 8 chunks, eight rows per block; the reference kernels' compiled
// size, flash_attn_fwd.metal:31).  Every swizzle is an involution in the chunk
// index, so a DMA lane fetches the logical chunk stored at its LDS position with the
// same function.
template <int D>
struct FaTile {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static constexpr int ROW = D * 2;            // bytes per row
  static constexpr int NCH = D / 8;            // 16-byte chunks per row
  static constexpr int RPB = 1024 / ROW;       // rows per 1 KB DMA block
  static constexpr int BYTES = FA_BK * ROW;    // one K or V block
  static constexpr int NBLK = BYTES / 1024;    // 1 KB DMA blocks per block
  static constexpr int NU = NBLK / 4;          // DMA instructions per wave per operand
  // Tiles read both ways (backward, and every d = 64 tile): chunk c of row r at
  // c ^ f(r).
  //   d = 128: f(r) = (r & 3) << 2 | (r >> 2) & 3.  f is a bijection on r & 15, so
  //     the 16 rows of a row read (16 lanes x 16 bytes) hit 16 distinct chunk
  //     positions; the 4 rows of a transposing read share bits 0-1 of f, so their
  //     32-byte chunk pairs still land in 4 distinct 64-byte groups.
  //   d = 64: a row is half of the 256-byte bank window, so rows r and r + 1 sit in
  //     opposite halves.  f(r) = ((r >> 1) & 1) << 2 | (r >> 2) & 3: over 16
  //     consecutive rows of one parity f takes all 8 values (row reads conflict
  //     free); of the 4 rows of a transposing read (4-aligned), the two of each
  //     parity differ in bit 2 of f, so their 64-byte segments (one half of the
  //     row's chunks, 32c .. 32c + 31 of d) land in opposite quarters of the window.
  __device__ static __forceinline__ int x_pos(int r, int c) {
    if constexpr (D == 128) return c ^ (((r & 3) << 2) | ((r >> 2) & 3));
    else return c ^ ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
  }
  // K tile [key][d], read as rows only: d = 128: chunk c of row r at c ^ (r & 15),
  // the 16 lanes of one ds_read_b128 phase reading 16 rows with distinct r & 15.
  __device__ static __forceinline__ int k_pos(int r, int c) {
    if constexpr (D == 128) return c ^ (r & 15);
    else return x_pos(r, c);
  }
  // V tile [key][d], read transposed only, its reads at rows krb + 4t + 16ks addressed
  // by one base per d block (the swizzle must not change with row bits 2 and up):
  // d = 128: chunk q of row r at q ^ ((r & 3) << 2), a transposing read touching 4
  // consecutive rows in 4 distinct 64-byte groups; d = 64: q ^ (((r >> 1) & 1) << 2),
  // rows r and r + 2 (same half of the bank window) in opposite quarters.
  __device__ static __forceinline__ int v_pos(int r, int q) {
    if constexpr (D == 128) return q ^ ((r & 3) << 2);
    else return q ^ (((r >> 1) & 1) << 2);
  }
  // DMA lane `lane` of 1 KB block u: tile row and LDS chunk position.
  __device__ static __forceinline__ int dma_row(int u, int lane) { return RPB * u + lane / NCH; }
  __device__ static __forceinline__ int dma_pos(int lane) { return lane % NCH; }
};

template <int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
    flash_fwd_kernel(FaParams p) {
  using Tl = FaTile<D>;
  constexpr int NS = D / 16;   // MFMA k-steps over d for S
  constexpr int NC = D / 32;   // 32-column blocks of d for O
  constexpr int STAGE = 2 * Tl::BYTES;  // K block then V block
  __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];
  const uint32_t lds0 = lds_addr(smem);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wave_u = uniform(wave);
  const int h32 = lane >> 5, l32 = lane & 31;

  // Heaviest query blocks first (causal work grows with the block index); the
  // heads of a KV group stay on one XCD, so they share K/V in its L2 (with B * nKV
  // a multiple of 8, every query block of the group runs there).
  const int BH = p.B * p.nH;
  const int lid = uniform(fa_xcd_spread(blockIdx.x, gridDim.x, p.group));
  const int qb = uniform(p.q_blocks - 1 - lid / BH);
  const int bh = uniform(lid - (lid / BH) * BH);
  const int b = uniform(bh / p.nH), h = uniform(bh - (bh / p.nH) * p.nH);
  const int kvh = uniform(h / p.group);
  const int T = p.T;
  const int q0 = qb * FA_BQ;
  const int qw = q0 + 32 * wave_u;  // first query row of this wave
  const int row = qw + l32;          // this lane's query row

  const __bf16* Qb = (const __bf16*)p.Q + ((int64_t)bh * T) * D;
  const __bf16* Kb = (const __bf16*)p.K + ((int64_t)(b * p.nKV + kvh) * T) * D;
  const __bf16* Vb = (const __bf16*)p.V + ((int64_t)(b * p.nKV + kvh) * T) * D;

  // Q fragments (second MFMA operand of S): row qw + l32, d = 16s + 8*h32 .. +7;
  // read from LDS before the first block.
  u32x4_t qf[NS];

  // Keys this workgroup needs: causal -> up to its last query row.
  const int kv_end = p.causal ? (q0 + FA_BQ < T ? q0 + FA_BQ : T) : T;
  const int nblk = uniform((kv_end + FA_BK - 1) / FA_BK);

  // DMA: wave w moves 1 KB blocks w*NU .. w*NU+NU-1 of the K and of the V block;
  // lane l of block u covers key row RPB*u + l/NCH, LDS chunk position l % NCH.
  uint32_t k_off[Tl::NU], v_off[Tl::NU];
#pragma unroll
  for (int u = 0; u < Tl::NU; ++u) {
    const int blk = wave * Tl::NU + u;
    const int r = Tl::dma_row(blk, lane), pos = Tl::dma_pos(lane);
    k_off[u] = (uint32_t)(r * Tl::ROW + 16 * Tl::k_pos(r, pos));  // k_pos is an involution
    v_off[u] = (uint32_t)(r * Tl::ROW + 16 * Tl::v_pos(r, pos));  // so is v_pos
  }
  const uint32_t dma_k = lds0 + (uint32_t)(wave_u * Tl::NU * 1024);
  const uint32_t dma_v = dma_k + Tl::BYTES;
  auto issue_block = [&](int j) __attribute__((always_inline)) {
    const int k0 = j * FA_BK;
    const uint32_t ext = (uint32_t)((T - k0) * Tl::ROW);  // keys >= T read as zero
    const __amdgpu_buffer_rsrc_t rk = scalar_rsrc(uniform(Kb + (int64_t)k0 * D), ext);
    const __amdgpu_buffer_rsrc_t rv = scalar_rsrc(uniform(Vb + (int64_t)k0 * D), ext);
    const uint32_t st = (uint32_t)((j & 1) * STAGE);
#pragma unroll
    for (int u = 0; u < Tl::NU; ++u) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rk, (__attribute__((address_space(3))) void*)(uintptr_t)(dma_k + st + (uint32_t)(u * 1024)), 16,
          (int)k_off[u], 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (__attribute__((address_space(3))) void*)(uintptr_t)(dma_v + st + (uint32_t)(u * 1024)), 16,
          (int)v_off[u], 0, 0, 0);
    }
  };

  // Fragment read addresses (stage 0).
  // K: first operand of S, row = key 32kb + perm(l32), d chunk 2s + h32.
  const uint32_t k_rd = (uint32_t)(fa_key_perm(l32) * Tl::ROW);
  // the swizzle of both halves' rows (32kb + perm(l32)) depends on row bits 0-3 only
  const int k_row = fa_key_perm(l32);
  // V: first operand of P V (rows = d, k = keys) through ds_read_b64_tr_b16: the
  // 16-lane group g reads key rows 8(g>>1) + (j>>2) (+4 for the second read) and
  // d columns 32c + 16(g&1) + 4(j&3) .. +3 and hands lane j the column 32c +
  // 16(g&1) + j with 4 consecutive keys.
  uint32_t v_rd[NC];
  {
    const int g = lane >> 4, jj = lane & 15;
    const int krb = 8 * (g >> 1) + (jj >> 2);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int col = 32 * c + 16 * (g & 1) + 4 * (jj & 3);
      v_rd[c] = (uint32_t)(Tl::BYTES + krb * Tl::ROW + 16 * Tl::v_pos(krb, col >> 3) + (col & 7) * 2);
    }
  }

  f32x16_t o[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[c][e] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;  // m_run in raw score units
  const float sl2 = p.scale_log2;
  // keys visible to this row: below row + 1 (causal) or below T
  const int lim = p.causal ? row + 1 : T;

  // One 64-key block; MASK: some key of the block is invisible to some row of the wave.
  auto block = [&](const int k0, const uint32_t st, auto MASK_c) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(MASK_c)::value;
    // ---- S = K Q^T for both 32-key halves ----
    f32x16_t sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[kb][e] = 0.0f;
    // all K fragments of the block first, so the MFMAs do not wait on each read
    u32x4_t kf[NS][2];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int c = 2 * s + h32;
        const uint32_t a = st + k_rd + (uint32_t)(32 * kb * Tl::ROW) + (uint32_t)(16 * Tl::k_pos(k_row, c));
        kf[s][kb] = *(const lds_u32x4_t*)(uintptr_t)a;
      }
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf[s][kb]),
                                                          __builtin_bit_cast(bf16x8_t, qf[s]),
                                                          sacc[kb], 0, 0, 0);

    // ---- online softmax, P fragments ----
    // sacc[kb][i], i = 4q + e, is key k0 + 32kb + 8*h32 + 16(q>>1) + 4(q&1) + e of
    // this lane's row.  The running max m is kept in raw score units; p =
    // 2^(s*c - m*c) with c = log2(e)/sqrt(d) is one FMA and one exp2 per score.
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int room = lim - (k0 + 32 * kb + 8 * h32);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if constexpr (MASK) {
          const int koff = 16 * ((i >> 2) >> 1) + 4 * ((i >> 2) & 1) + (i & 3);
          sacc[kb][i] = koff < room ? sacc[kb][i] : -INFINITY;
        }
        mx = fmaxf(mx, sacc[kb][i]);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // Conditional rescaling: a row keeps its reference max until a block raises
    // it by more than FA_TAU (in log2 units of p), so p stays below 2^FA_TAU and O
    // is rescaled only on the blocks where some row of the wave moves its
    // reference -- the result is the same for any reference max, only the
    // rounding of intermediate values differs.  A row with no visible key yet
    // (m = -inf) has O = 0 and l = 0 and just takes the new max.
    const float m_old = m_run;
    const bool fresh = m_old == -INFINITY;
    const bool raise = !fresh && (mx - m_old) * sl2 > FA_TAU;
    const float m_ref = (fresh || raise) ? mx : m_old;
    if (__any(raise)) {
      const float alpha = raise ? __builtin_amdgcn_exp2f((m_old - m_ref) * sl2) : 1.0f;
      l_run *= alpha;
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[c][e] *= alpha;
    }
    m_run = m_ref;
    // rows with no visible key so far (non-causal tail rows) stay at m = -inf;
    // their p is 2^(-inf) = 0
    const float nmc = m_ref == -INFINITY ? 0.0f : -m_ref * sl2;
    float sum = 0.0f;
    u32x4_t pf[4];
    // k-step ks covers keys 16ks .. 16ks+15: registers 8(ks&1) .. +7 of half ks>>1
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int kb = ks >> 1, base = 8 * (ks & 1);
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) {
        const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][base + 2 * w2], sl2, nmc));
        const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][base + 2 * w2 + 1], sl2, nmc));
        sum += e0 + e1;
        pf[ks][w2] = pack_bf16x2(e0, e1);
      }
    }
    l_run += sum;

    // ---- O += P V ----
    static_for<4>([&](auto ks_c) __attribute__((always_inline)) {
      constexpr int ks = decltype(ks_c)::value;
      u32x4_t vf[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        static_for<2>([&](auto t_c) __attribute__((always_inline)) {
          constexpr int t = decltype(t_c)::value;
          u32x2_t w2 = {0u, 0u};
#if defined(__HIP_DEVICE_COMPILE__)
          // inline asm: the builtin would also wait for the K/V DMA in flight
          asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                       : "=v"(w2)
                       : "v"(st + v_rd[c]), "i"((16 * ks + 4 * t) * Tl::ROW));
#endif
          vf[c][2 * t] = w2[0];
          vf[c][2 * t + 1] = w2[1];
        });
      }
      // The asm results are only valid after lgkmcnt(0), which the compiler does
      // not know: the scheduling barrier keeps the MFMAs below the wait.
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < NC; ++c)
        o[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vf[c]),
                                                       __builtin_bit_cast(bf16x8_t, pf[ks]), o[c],
                                                       0, 0, 0);
    });
  };

  // Blocks 0 .. jd-1 are visible to every row of the wave (no mask); the rest
  // hold the causal diagonal or the key tail.  Both loops run one ring step per
  // block, so every wave passes the same barriers.
  const int jd = uniform(p.causal ? (qw + 1) / FA_BK : T / FA_BK);
  const int j_split = jd < nblk ? jd : nblk;
  auto ring_step = [&](int j) __attribute__((always_inline)) {
    wait_vmcnt<0>();     // this wave's share of block j landed
    lds_ring_barrier();  // every share landed; every wave is done with block j-1
    if (j + 1 < nblk) issue_block(j + 1);
    return lds0 + (uint32_t)((j & 1) * STAGE);
  };
  // Q goes global -> LDS stage 1 as whole 256-byte rows (the K tile's layout and DMA
  // offsets, 64 rows per half; rows past T read as zero), together with block 0.
  // Each wave then reads its 32 rows' fragments; ring_step(0)'s barrier (after
  // lgkmcnt(0)) frees stage 1 for block 1.  (Per-lane 16-byte global loads of the
  // fragments: about 1 us slower at configuration 4.)
  {
    const uint32_t dst = lds0 + (uint32_t)STAGE + (uint32_t)(wave_u * Tl::NU * 1024);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int r0 = q0 + 64 * half;
      const uint32_t ext = r0 < T ? (uint32_t)((T - r0) * Tl::ROW) : 0u;
      const __amdgpu_buffer_rsrc_t rq = scalar_rsrc(uniform(Qb + (int64_t)(r0 < T ? r0 : 0) * D), ext);
#pragma unroll
      for (int u = 0; u < Tl::NU; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rq, (__attribute__((address_space(3))) void*)(uintptr_t)(dst + (uint32_t)(half * Tl::BYTES + u * 1024)),
            16, (int)k_off[u], 0, 0, 0);
    }
  }
  if (nblk > 0) issue_block(0);
  wait_vmcnt<0>();
  lds_ring_barrier();
  {
    const int qr = 32 * (wave_u & 1) + l32;  // row within the wave's 64-row half
    const uint32_t qbase = lds0 + (uint32_t)(STAGE + (wave_u >> 1) * Tl::BYTES + qr * Tl::ROW);
#pragma unroll
    for (int s = 0; s < NS; ++s)
      qf[s] = *(const lds_u32x4_t*)(uintptr_t)(qbase + (uint32_t)(16 * Tl::k_pos(qr, 2 * s + h32)));
  }
  for (int j = 0; j < j_split; ++j) {
    const uint32_t st = ring_step(j);
    block(j * FA_BK, st, std::false_type{});
  }
  for (int j = j_split; j < nblk; ++j) {
    const uint32_t st = ring_step(j);
    if (p.causal && j * FA_BK > qw + 31) continue;  // above every row of this wave
    block(j * FA_BK, st, std::true_type{});
  }

  // ---- normalise and store ----
  // O goes out through LDS so that NCH lanes store one whole row: each wave writes
  // its 32 x d tile to a region in the K tile's layout (k_pos) and reads it back as
  // whole rows (16 lanes per 256-byte row, or 8 per 128-byte row).  The barrier
  // keeps the regions, which overlap stage 0 of the ring, from other waves' reads of
  // their last block.  (8-byte stores straight from the accumulators: 1-1.5 us
  // slower at configuration 4.)
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  __syncthreads();
  const uint32_t ob = lds0 + (uint32_t)(wave_u * 32 * Tl::ROW);
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int ch = 4 * c + q;  // chunk of d = 32c + 8q + 4*h32 .. +3, half h32
      const uint32_t a = ob + (uint32_t)(l32 * Tl::ROW + Tl::k_pos(l32, ch) * 16 + h32 * 8);
      *(__attribute__((address_space(3))) u32x2_t*)(uintptr_t)a =
          u32x2_t{pack_bf16x2(o[c][4 * q] * inv, o[c][4 * q + 1] * inv),
                  pack_bf16x2(o[c][4 * q + 2] * inv, o[c][4 * q + 3] * inv)};
    }
  // read back as whole rows: NCH lanes per row, 64 / NCH rows per read
  const int oj = lane % Tl::NCH;
#pragma unroll
  for (int i = 0; i < 32 * Tl::NCH / 64; ++i) {
    const int rr = (64 / Tl::NCH) * i + lane / Tl::NCH;
    const u32x4_t v = *(const __attribute__((address_space(3))) u32x4_t*)(uintptr_t)(
        ob + (uint32_t)(rr * Tl::ROW + Tl::k_pos(rr, oj) * 16));
    const int orow_i = qw + rr;
    if (orow_i < T) {
      uint16_t* orow = (uint16_t*)p.O + (p.o_bthd ? ((int64_t)(b * T + orow_i) * p.nH + h) * D
                                                  : ((int64_t)bh * T + orow_i) * D);
      // non-temporal: O is read again only by the backward (forward 64-66 -> 62-63 us, one box)
      __builtin_nontemporal_store(v, (u32x4_t*)(orow + 8 * oj));
    }
  }
  if (row < T && p.lse && h32 == 0)
    p.lse[(int64_t)bh * T + row] = l_tot > 0.0f ? (m_run * sl2 + __log2f(l_tot)) * 0.69314718055994531f
                                               : -INFINITY;
}

// Lane-row reads of a 32-row half of a [row][d] tile read with the bit-2/3 swapped
// row order: rows 32*half + perm(l32), d chunk 2s + h32.  Transposing reads of the
// same tile: rows 16ks + 8*(g>>1) + (j>>2) (+4), d columns 32c + 16(g&1) + 4(j&3).
template <int D>
struct FaReads {
  uint32_t row_base;  // perm(l32) * ROW
  int row_lo;         // perm(l32): x_pos of rows 32*half + perm(l32) depends on bits 0-3
  // transposing-read bases for the rows krb (first read) and krb + 4 (second): the
  // swizzle depends on row bits 2-3, so the two reads need their own base
  uint32_t tr[D / 32][2];
  __device__ __forceinline__ void init(int lane) {
    using Tl = FaTile<D>;
    const int l32 = lane & 31;
    row_base = (uint32_t)(fa_key_perm(l32) * Tl::ROW);
    row_lo = fa_key_perm(l32);
    const int g = lane >> 4, jj = lane & 15;
    const int krb = 8 * (g >> 1) + (jj >> 2);
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
      const int col = 32 * c + 16 * (g & 1) + 4 * (jj & 3);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int r = krb + 4 * t;
        tr[c][t] = (uint32_t)(r * Tl::ROW + 16 * Tl::x_pos(r, col >> 3) + (col & 7) * 2);
      }
    }
  }
  // 16 bytes of row-read fragment (half, k-step s) of the tile at LDS address t
  __device__ __forceinline__ u32x4_t row(uint32_t t, int half, int s, int h32) const {
    using Tl = FaTile<D>;
    const int c = 2 * s + h32;
    // rows 32*half + perm(l32): the swizzle is row_lo's for both halves
    const uint32_t a = t + row_base + (uint32_t)(32 * half * Tl::ROW) + (uint32_t)(16 * Tl::x_pos(row_lo, c));
    return *(const lds_u32x4_t*)(uintptr_t)a;
  }
};

// Transposing fragment (d block c, key/query k-step KS) of the tile at LDS address
// t: two ds_read_b64_tr_b16.  The caller waits lgkmcnt(0) and fences the scheduler
// before using the result.
template <int D, int KS>
__device__ __forceinline__ u32x4_t fa_tr_frag(uint32_t t, const uint32_t* tr) {
  [[maybe_unused]] constexpr int ROW = FaTile<D>::ROW;
  u32x4_t out = {0u, 0u, 0u, 0u};
  static_for<2>([&](auto t_c) __attribute__((always_inline)) {
    constexpr int TT = decltype(t_c)::value;
    u32x2_t w2 = {0u, 0u};
#if defined(__HIP_DEVICE_COMPILE__)
    // rows 16KS + krb + 4TT: 16KS leaves the swizzle unchanged, an immediate offset
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                 : "=v"(w2)
                 : "v"(t + tr[TT]), "i"(16 * KS * ROW));
#endif
    out[2 * TT] = w2[0];
    out[2 * TT + 1] = w2[1];
  });
  return out;
}

__device__ __forceinline__ void fa_lds_fence() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_sched_barrier(0);
}

// One 16-byte DMA of a [row][d] tile: lane l of 1 KB block u covers row RPB*u +
// l/NCH, LDS position l % NCH (dual swizzle), reading row `r` of a matrix whose rows
// are `stride` bytes apart.
template <int D>
__device__ __forceinline__ uint32_t fa_dma_off(int u, int lane, int stride) {
  using Tl = FaTile<D>;
  const int r = Tl::dma_row(u, lane), pos = Tl::dma_pos(lane);
  return (uint32_t)(r * stride + 16 * Tl::x_pos(r, pos));  // x_pos is an involution in c
}

// dQ for 128 query rows of one (batch, head): recompute S = Q K^T and P from the
// forward's log-sum-exp, dP = dO V^T, dS = P (dP - D), dQ = scale * dS K, with the
// K/V blocks streamed like the forward's.  D = rowsum(dO O) comes from the D kernel,
// launched before this one.
template <int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
    flash_bwd_dq_kernel(FbParams p) {
  using Tl = FaTile<D>;
  using Rd = FaReads<D>;
  constexpr int NS = D / 16, NC = D / 32;
  constexpr int STAGE = 2 * Tl::BYTES;
  __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];
  const uint32_t lds0 = lds_addr(smem);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wave_u = uniform(wave);
  const int h32 = lane >> 5, l32 = lane & 31;

  const int BH = p.B * p.nH;
  const int lid = uniform(fa_xcd_spread(blockIdx.x, gridDim.x, p.group));  // as the forward
  const int qb = uniform(p.q_blocks - 1 - lid / BH);
  const int bh = uniform(lid - (lid / BH) * BH);
  const int b = uniform(bh / p.nH), h = uniform(bh - (bh / p.nH) * p.nH);
  const int kvh = uniform(h / p.group);
  const int T = p.T;
  const int q0 = qb * FA_BQ;
  const int qw = q0 + 32 * wave_u;
  const int row = qw + l32;
  const bool live = row < T;

  const __bf16* Qb = (const __bf16*)p.Q + ((int64_t)bh * T) * D;
  const __bf16* Kb = (const __bf16*)p.K + ((int64_t)(b * p.nKV + kvh) * T) * D;
  const __bf16* Vb = (const __bf16*)p.V + ((int64_t)(b * p.nKV + kvh) * T) * D;
  const int64_t orow = p.o_bthd ? ((int64_t)(b * T + row) * p.nH + h) * D : ((int64_t)bh * T + row) * D;

  // Q and dO fragments (second MFMA operands), the row's D (from the D kernel, which
  // runs first) and log-sum-exp.
  u32x4_t qf[NS], gf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int dd = 16 * s + 8 * h32;
    if (live) {
      qf[s] = *(const u32x4_t*)(Qb + (int64_t)row * D + dd);
      gf[s] = *(const u32x4_t*)((const __bf16*)p.dO + orow + dd);
    } else {
      qf[s] = u32x4_t{0u, 0u, 0u, 0u};
      gf[s] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }
  const float dsum = live ? p.delta[(int64_t)bh * T + row] : 0.0f;
  const float lse2 = live ? p.lse[(int64_t)bh * T + row] * 1.4426950408889634f : 0.0f;
  const float sl2 = p.scale_log2;

  const int kv_end = p.causal ? (q0 + FA_BQ < T ? q0 + FA_BQ : T) : T;
  const int nblk = uniform((kv_end + FA_BK - 1) / FA_BK);

  // DMA of the K and V blocks (dual swizzle: both are read as rows and transposed)
  uint32_t offs[Tl::NU];
#pragma unroll
  for (int u = 0; u < Tl::NU; ++u) offs[u] = fa_dma_off<D>(wave * Tl::NU + u, lane, Tl::ROW);
  const uint32_t dma_k = lds0 + (uint32_t)(wave_u * Tl::NU * 1024);
  const uint32_t dma_v = dma_k + Tl::BYTES;
  auto issue_block = [&](int j) __attribute__((always_inline)) {
    const int k0 = j * FA_BK;
    const uint32_t ext = (uint32_t)((T - k0) * Tl::ROW);
    const __amdgpu_buffer_rsrc_t rk = scalar_rsrc(uniform(Kb + (int64_t)k0 * D), ext);
    const __amdgpu_buffer_rsrc_t rv = scalar_rsrc(uniform(Vb + (int64_t)k0 * D), ext);
    const uint32_t st = (uint32_t)((j & 1) * STAGE);
#pragma unroll
    for (int u = 0; u < Tl::NU; ++u) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rk, (__attribute__((address_space(3))) void*)(uintptr_t)(dma_k + st + (uint32_t)(u * 1024)), 16,
          (int)offs[u], 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (__attribute__((address_space(3))) void*)(uintptr_t)(dma_v + st + (uint32_t)(u * 1024)), 16,
          (int)offs[u], 0, 0, 0);
    }
  };
  Rd rd;
  rd.init(lane);

  f32x16_t dq[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) dq[c][e] = 0.0f;
  const int lim = p.causal ? row + 1 : T;

  auto block = [&](const int k0, const uint32_t st, auto MASK_c) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(MASK_c)::value;
    const uint32_t tk = st, tv = st + Tl::BYTES;
    f32x16_t sacc[2], pacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[kb][e] = pacc[kb][e] = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4_t kf = rd.row(tk, kb, s, h32);
        const u32x4_t vf = rd.row(tv, kb, s, h32);
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf),
                                                          __builtin_bit_cast(bf16x8_t, qf[s]),
                                                          sacc[kb], 0, 0, 0);
        pacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vf),
                                                          __builtin_bit_cast(bf16x8_t, gf[s]),
                                                          pacc[kb], 0, 0, 0);
      }
    // register i of half kb: key k0 + 32kb + 8*h32 + 16((i>>2)>>1) + 4((i>>2)&1) + (i&3)
    u32x4_t df[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int kb = ks >> 1, base = 8 * (ks & 1);
      const int room = lim - (k0 + 32 * kb + 8 * h32);
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) {
        float ds[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int i = base + 2 * w2 + u;
          float x = __builtin_fmaf(sacc[kb][i], sl2, -lse2);
          if constexpr (MASK) {
            const int koff = 16 * ((i >> 2) >> 1) + 4 * ((i >> 2) & 1) + (i & 3);
            x = koff < room ? x : -INFINITY;
          }
          ds[u] = __builtin_amdgcn_exp2f(x) * (pacc[kb][i] - dsum);
        }
        df[ks][w2] = pack_bf16x2(ds[0], ds[1]);
      }
    }
    // dQ += dS K: first operand K^T through the transposing read of the K tile
    static_for<4>([&](auto ks_c) __attribute__((always_inline)) {
      constexpr int KS = decltype(ks_c)::value;
      u32x4_t kt[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) kt[c] = fa_tr_frag<D, KS>(tk, rd.tr[c]);
      fa_lds_fence();
#pragma unroll
      for (int c = 0; c < NC; ++c)
        dq[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kt[c]),
                                                        __builtin_bit_cast(bf16x8_t, df[KS]), dq[c],
                                                        0, 0, 0);
    });
  };

  const int jd = uniform(p.causal ? (qw + 1) / FA_BK : T / FA_BK);
  const int j_split = jd < nblk ? jd : nblk;
  auto ring_step = [&](int j) __attribute__((always_inline)) {
    wait_vmcnt<0>();
    lds_ring_barrier();
    if (j + 1 < nblk) issue_block(j + 1);
    return lds0 + (uint32_t)((j & 1) * STAGE);
  };
  if (nblk > 0) issue_block(0);
  for (int j = 0; j < j_split; ++j) {
    const uint32_t st = ring_step(j);
    block(j * FA_BK, st, std::false_type{});
  }
  for (int j = j_split; j < nblk; ++j) {
    const uint32_t st = ring_step(j);
    if (p.causal && j * FA_BK > qw + 31) continue;
    block(j * FA_BK, st, std::true_type{});
  }

  if (live) {
    uint16_t* out = (uint16_t*)p.dQ + ((int64_t)bh * T + row) * D;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int d = 32 * c + 8 * q + 4 * h32;
        *(u32x2_t*)(out + d) = u32x2_t{pack_bf16x2(dq[c][4 * q] * p.scale, dq[c][4 * q + 1] * p.scale),
                                       pack_bf16x2(dq[c][4 * q + 2] * p.scale, dq[c][4 * q + 3] * p.scale)};
      }
  }
}

// dK and dV for 128 keys of one (batch, KV head): the query tiles (64 rows) of
// every query head of the KV group stream through a two-stage LDS ring (Q, dO,
// the forward's log-sum-exp and D); S^T = K Q^T and dP^T = V dO^T with one lane
// per key, P^T and dS^T = P^T (dP^T - D) in registers, then dV += P^T dO and
// dK += scale * dS^T Q.  The KV-group reduction (Attention.cpp:332,344-345) is the
// loop over the group's heads.  DS: also store dS^T (bf16, [B, nH, key, query]) for
// dQ = scale * dS K as a batched GEMM.
//
// Eight waves, two per SIMD: waves w and w + 4 hold the same 32 keys and take the
// first and second 32-query half of every tile, so one wave's softmax (VALU) runs
// under the other's MFMAs.  The 128 keys' K and V tiles stay in LDS for the whole
// unit and are read as MFMA fragments each tile, which leaves a wave its 32 x d dK
// and dV accumulators within the 256 registers of two waves per SIMD; at the end
// the halves are added in LDS (first half + second half).  Configuration 4's
// dK/dV: 117 us against 128 us for four waves (one per SIMD, K and V fragments in
// registers, the two halves interleaved in one wave).
template <int D, bool DS>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
    flash_bwd_dkdv_kernel(FbParams p) {
  using Tl = FaTile<D>;
  using Rd = FaReads<D>;
  constexpr int NS = D / 16, NC = D / 32;
  constexpr int QT = FA_BK;                          // query rows per tile
  constexpr int KVB = 128 * Tl::ROW;                 // one 128-key K or V tile
  constexpr int NU = Tl::NBLK / 8;                   // 1 KB DMA blocks per wave per 64-row tile
  constexpr int NUK = KVB / 1024 / 8;                // ... per 128-key tile
  constexpr int STAGE = 2 * Tl::BYTES + 2 * QT * 4;  // Q, dO, lse, D
  constexpr int RING = 2 * KVB;                      // the ring follows K and V
  static_assert(NU >= 1 && NUK >= 1, "whole DMA blocks per wave");
  __shared__ __attribute__((aligned(16))) char smem[RING + 2 * STAGE];
  const uint32_t lds0 = lds_addr(smem);
  const uint32_t lk = lds0, lv = lds0 + KVB, lr = lds0 + RING;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wave_u = uniform(wave);
  const int wq = uniform(wave_u & 3), qh = uniform(wave_u >> 2);
  const int h32 = lane >> 5, l32 = lane & 31;

  // Work unit: with a schedule, unit u (largest first) of every (batch, KV head) in
  // turn, so each XCD (workgroups b mod 8) gets an even share of every size;
  // without, one key block per workgroup, the ones with the most query tiles
  // (causal: the first) first, spread over the XCDs the same way.
  const int BKV = p.B * p.nKV;
  int kbi, bkv, slot = -1, ib = 0, ie = -1;
  if (p.n_units) {
    const int u = uniform((int)blockIdx.x / BKV);
    bkv = uniform((int)blockIdx.x - u * BKV);
    const uint32_t uk = uniform(p.unit_kbi[u]), ur = uniform(p.unit_range[u]);
    kbi = (int)(uk & 0xffffu);
    slot = (int)(uk >> 16) - 1;
    ib = (int)(ur & 0xffffu);
    ie = (int)(ur >> 16);
  } else {
    const int lid = uniform(fa_xcd_spread(blockIdx.x, gridDim.x, 1));
    kbi = uniform(lid / BKV);
    bkv = uniform(lid - kbi * BKV);
  }
  const int b = uniform(bkv / p.nKV), kvh = uniform(bkv - (bkv / p.nKV) * p.nKV);
  const int T = p.T;
  const int k0 = kbi * 128;
  const int kw = k0 + 32 * wq;
  const int key = kw + l32;
  const bool live = key < T;

  const __bf16* Kb = (const __bf16*)p.K + ((int64_t)bkv * T) * D;
  const __bf16* Vb = (const __bf16*)p.V + ((int64_t)bkv * T) * D;
  // K and V tiles of the 128 keys into LDS (keys past T read as zero)
  {
    const uint32_t ext = (uint32_t)((T - k0) * Tl::ROW);
    const __amdgpu_buffer_rsrc_t rk = scalar_rsrc(uniform(Kb + (int64_t)k0 * D), ext);
    const __amdgpu_buffer_rsrc_t rv = scalar_rsrc(uniform(Vb + (int64_t)k0 * D), ext);
#pragma unroll
    for (int u = 0; u < NUK; ++u) {
      const int blk = wave * NUK + u;
      const uint32_t off = fa_dma_off<D>(blk, lane, Tl::ROW);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rk, (__attribute__((address_space(3))) void*)(uintptr_t)(lk + (uint32_t)(blk * 1024)), 16, (int)off,
          0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (__attribute__((address_space(3))) void*)(uintptr_t)(lv + (uint32_t)(blk * 1024)), 16, (int)off,
          0, 0, 0);
    }
  }
  // Fragment s (d chunk 2s + h32) of this lane's key row in the K or V tile.
  const int krow = 32 * wq + l32;
  auto kv_frag = [&](uint32_t t, int s) __attribute__((always_inline)) {
    const uint32_t a = t + (uint32_t)(krow * Tl::ROW + 16 * Tl::x_pos(krow, 2 * s + h32));
    return *(const lds_u32x4_t*)(uintptr_t)a;
  };

  const int nqt = (T + QT - 1) / QT;
  const int qt0 = uniform(p.causal ? k0 / QT : 0);
  const int per_h = uniform(nqt - qt0);
  const int total = uniform(per_h > 0 ? per_h * p.group : 0);
  if (ie < 0) ie = total;
  const int go_stride = (p.o_bthd ? p.nH * D : D) * 2;

  uint32_t q_off[NU], g_off[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    q_off[u] = fa_dma_off<D>(wave * NU + u, lane, Tl::ROW);
    g_off[u] = fa_dma_off<D>(wave * NU + u, lane, go_stride);
  }
  const uint32_t dma_q = lr + (uint32_t)(wave_u * NU * 1024);
  const uint32_t dma_g = dma_q + Tl::BYTES;
  const uint32_t dma_l = lr + 2 * Tl::BYTES + (uint32_t)(wave_u * QT * 4);  // waves 0, 1
  auto tile_at = [&](int it, int& h, int& q0) __attribute__((always_inline)) {
    const int hh = it / per_h;
    h = kvh * p.group + hh;
    q0 = (qt0 + (it - hh * per_h)) * QT;
  };
  auto issue = [&](int it) __attribute__((always_inline)) {
    int h, q0;
    tile_at(it, h, q0);
    const int bh = b * p.nH + h;
    const int rows = T - q0;
    const __amdgpu_buffer_rsrc_t rq =
        scalar_rsrc(uniform((const __bf16*)p.Q + ((int64_t)bh * T + q0) * D), (uint32_t)(rows * Tl::ROW));
    const int64_t g0 = p.o_bthd ? ((int64_t)(b * T + q0) * p.nH + h) * D : ((int64_t)bh * T + q0) * D;
    const __amdgpu_buffer_rsrc_t rg = scalar_rsrc(uniform((const __bf16*)p.dO + g0),
                                                  (uint32_t)((rows - 1) * go_stride + Tl::ROW));
    const uint32_t st = (uint32_t)((it & 1) * STAGE);
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rq, (__attribute__((address_space(3))) void*)(uintptr_t)(dma_q + st + (uint32_t)(u * 1024)), 16,
          (int)q_off[u], 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rg, (__attribute__((address_space(3))) void*)(uintptr_t)(dma_g + st + (uint32_t)(u * 1024)), 16,
          (int)g_off[u], 0, 0, 0);
    }
    if (wave_u < 2) {  // wave 0: log-sum-exp, wave 1: D, 4 bytes per lane
      const float* src = (wave_u == 0 ? p.lse : p.delta) + (int64_t)bh * T + q0;
      const __amdgpu_buffer_rsrc_t rl = scalar_rsrc(uniform(src), (uint32_t)(rows * 4));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rl, (__attribute__((address_space(3))) void*)(uintptr_t)(dma_l + st), 4, lane * 4, 0, 0, 0);
    }
  };
  Rd rd;
  rd.init(lane);

  f32x16_t dk[NC], dv[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) dk[c][e] = dv[c][e] = 0.0f;
  const float sl2 = p.scale_log2;

  // dS^T rows of this lane's key: registers 8kk .. 8kk+7 of the wave's half hold 8
  // consecutive queries, stored as one 16-byte buffer store, 2 per wave and tile.
  // Lanes l and l + 32 hold the same key, so the two halves' waves fill each key's
  // 128-byte line of a tile.  Lanes past the last key, and runs past the last query
  // (T % 8 == 0, so a run is all in or all out), get an offset beyond the tile
  // descriptor's range, which the hardware drops: every wave issues exactly 2 stores
  // per tile, and ring_step's wait counts them (vmcnt retires in issue order on
  // gfx9-family parts).
  const uint32_t ds_lane = live ? (uint32_t)(key * T + 8 * h32) * 2u : 0x80000000u;
  auto store_ds = [&](int bh, int q0, auto&& run) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rs =
        scalar_rsrc(uniform((const uint16_t*)p.dsT + (int64_t)bh * T * T + q0),
                    (uint32_t)(((int64_t)T * T - q0) * 2));
    const int lim = T - q0 - 8 * h32;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int c = 32 * qh + 16 * kk;
      const uint32_t off = c < lim ? ds_lane : 0x80000000u;
      __builtin_amdgcn_raw_buffer_store_b128(run(kk), rs, off + 2 * c, 0, 0);
    }
  };
  // One query tile, this wave's 32-query half qh: register i of sacc / pacc is query
  // q0 + 32qh + 8*h32 + 16((i>>2)>>1) + 4((i>>2)&1) + (i&3) of this lane's key.
  auto block = [&](const int q0, const int bh, const uint32_t st, auto MASK_c) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(MASK_c)::value;
    const uint32_t tq = st, tg = st + Tl::BYTES, tl = st + 2 * Tl::BYTES, td = tl + QT * 4;
    f32x16_t sacc, pacc;
#pragma unroll
    for (int e = 0; e < 16; ++e) sacc[e] = pacc[e] = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const u32x4_t qr = rd.row(tq, qh, s, h32);
      const u32x4_t gr = rd.row(tg, qh, s, h32);
      const u32x4_t kr = kv_frag(lk, s);
      const u32x4_t vr = kv_frag(lv, s);
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, qr),
                                                     __builtin_bit_cast(bf16x8_t, kr), sacc, 0, 0, 0);
      pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, gr),
                                                     __builtin_bit_cast(bf16x8_t, vr), pacc, 0, 0, 0);
    }
    // P and dS = P (dP - D) of the half's two k-steps, as bf16 pairs
    u32x4_t pf[2], df[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int base = 8 * kk;
      const int tix = 32 * qh + 8 * h32 + 16 * kk;  // tile index of register `base`
      const f32x4_t l0 = *(const __attribute__((address_space(3))) f32x4_t*)(uintptr_t)(tl + 4 * tix);
      const f32x4_t l1 = *(const __attribute__((address_space(3))) f32x4_t*)(uintptr_t)(tl + 4 * (tix + 4));
      const f32x4_t d0 = *(const __attribute__((address_space(3))) f32x4_t*)(uintptr_t)(td + 4 * tix);
      const f32x4_t d1 = *(const __attribute__((address_space(3))) f32x4_t*)(uintptr_t)(td + 4 * (tix + 4));
      const int need = key - (q0 + tix);
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) {
        float pv[2], dsv[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int r = 2 * w2 + u;
          const float lsev = r < 4 ? l0[r & 3] : l1[r & 3];
          const float dlt = r < 4 ? d0[r & 3] : d1[r & 3];
          float x = __builtin_fmaf(sacc[base + r], sl2, -lsev * 1.4426950408889634f);
          if constexpr (MASK) x = r >= need ? x : -INFINITY;
          pv[u] = __builtin_amdgcn_exp2f(x);
          dsv[u] = pv[u] * (pacc[base + r] - dlt);
        }
        pf[kk][w2] = pack_bf16x2(pv[0], pv[1]);
        df[kk][w2] = pack_bf16x2(dsv[0], dsv[1]);
      }
    }
    if constexpr (DS) store_ds(bh, q0, [&](int kk) { return df[kk]; });
    // dV += P^T dO, dK += dS^T Q over the half's k-steps (query rows 32qh + 16kk ..)
    const uint32_t hq = (uint32_t)(32 * qh * Tl::ROW);
    // The 8 (k-step, 32-column block) pairs in turn, the next pair's 4 transposing
    // reads issued before this pair's MFMAs: LDS returns in order, so lgkmcnt(4)
    // leaves exactly the next pair's reads in flight.
    u32x4_t gt[2], qt[2];
    gt[0] = fa_tr_frag<D, 0>(tg + hq, rd.tr[0]);
    qt[0] = fa_tr_frag<D, 0>(tq + hq, rd.tr[0]);
    static_for<2 * NC>([&](auto i_c) __attribute__((always_inline)) {
      constexpr int I = decltype(i_c)::value, KK = I / NC, C = I % NC, B = I & 1;
      if constexpr (I + 1 < 2 * NC) {
        constexpr int KN = (I + 1) / NC, CN = (I + 1) % NC;
        gt[B ^ 1] = fa_tr_frag<D, KN>(tg + hq, rd.tr[CN]);
        qt[B ^ 1] = fa_tr_frag<D, KN>(tq + hq, rd.tr[CN]);
        __builtin_amdgcn_s_waitcnt(0xC07F | (4 << 8));  // lgkmcnt(4)
      } else {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      }
      __builtin_amdgcn_sched_barrier(0);
      dv[C] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, gt[B]),
                                                      __builtin_bit_cast(bf16x8_t, pf[KK]), dv[C], 0, 0, 0);
      dk[C] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, qt[B]),
                                                      __builtin_bit_cast(bf16x8_t, df[KK]), dk[C], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // Per head: the first n_diag tiles may hold queries before some of this wave's keys
  // (causal mask); the rest are visible whole.  Separate loops keep the accumulators
  // in place across iterations.
  const int n_diag = uniform(p.causal ? (per_h < 2 ? per_h : 2) : 0);
  auto ring_step = [&](int it) __attribute__((always_inline)) {
    if (DS && it > ib) wait_vmcnt<2>();  // the last tile's two dS^T stores stay in flight
    else wait_vmcnt<0>();
    lds_ring_barrier();
    if (it + 1 < ie) issue(it + 1);
    return lr + (uint32_t)((it & 1) * STAGE);
  };
  if (ib < ie) issue(ib);
  int it = 0;
  for (int hh = 0; hh < p.group; ++hh) {
    const int bh = uniform(b * p.nH + kvh * p.group + hh);
    for (int t = 0; t < n_diag; ++t, ++it) {
      if (it < ib || it >= ie) continue;
      const uint32_t st = ring_step(it);
      const int q0 = uniform((qt0 + t) * QT);
      // A tile wholly above this wave's keys: skipped without dS^T; with it, the
      // masked block writes its zeros (the dQ GEMM reads whole K tiles around the
      // diagonal).  Zeros from the block itself keep the loop to one path, which
      // the register allocator needs here.
      if (!DS && q0 + QT - 1 < kw) continue;
      block(q0, bh, st, std::true_type{});
    }
    for (int t = n_diag; t < per_h; ++t, ++it) {
      if (it < ib || it >= ie) continue;
      const uint32_t st = ring_step(it);
      block(uniform((qt0 + t) * QT), bh, st, std::false_type{});
    }
  }

  // Halves added in LDS: wave (wq, 0) finishes dK, wave (wq, 1) finishes dV, each as
  // first half + second half.
  wait_vmcnt<0>();
  __syncthreads();
  f32x4_t* xb = reinterpret_cast<f32x4_t*>(smem);
  auto slot_of = [&](int w, int c, int q) __attribute__((always_inline)) {
    return ((w * NC + c) * 4 + q) * 64 + lane;
  };
  // wave (wq, 1) sends its dK half to slots of wq; wave (wq, 0) sends its dV half to
  // slots of 4 + wq
  auto send = [&](f32x16_t (&src)[NC], int w) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        xb[slot_of(w, c, q)] = f32x4_t{src[c][4 * q], src[c][4 * q + 1], src[c][4 * q + 2], src[c][4 * q + 3]};
  };
  if (qh) send(dk, wq);
  else send(dv, 4 + wq);
  __syncthreads();
  if (qh == 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4_t o = xb[slot_of(wq, c, q)];
#pragma unroll
        for (int e = 0; e < 4; ++e) dk[c][4 * q + e] = dk[c][4 * q + e] + o[e];  // half 0 + half 1
      }
  } else {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4_t o = xb[slot_of(4 + wq, c, q)];
#pragma unroll
        for (int e = 0; e < 4; ++e) dv[c][4 * q + e] = o[e] + dv[c][4 * q + e];
      }
  }

  // wave (wq, 0) writes dK, wave (wq, 1) writes dV
  const int lrow = krow * D;
  auto write = [&](const f32x16_t (&res)[NC], int half, float* part_half, uint16_t* o, float sc)
      __attribute__((always_inline)) {
    if (!live) return;
    if (slot >= 0) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *(f32x4_t*)(part_half + lrow + 32 * c + 8 * q + 4 * h32) =
              f32x4_t{res[c][4 * q], res[c][4 * q + 1], res[c][4 * q + 2], res[c][4 * q + 3]};
    } else {
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *(u32x2_t*)(o + lrow + 32 * c + 8 * q + 4 * h32) =
              u32x2_t{pack_bf16x2(res[c][4 * q] * sc, res[c][4 * q + 1] * sc),
                      pack_bf16x2(res[c][4 * q + 2] * sc, res[c][4 * q + 3] * sc)};
    }
    (void)half;
  };
  float* pk = slot >= 0 ? uniform(p.part + ((int64_t)bkv * p.n_slots + slot) * 2 * 128 * D) : nullptr;
  const int64_t obase = ((int64_t)bkv * T + k0) * D;
  if (qh == 0) write(dk, 0, pk, (uint16_t*)p.dK + obase, p.scale);
  else write(dv, 1, pk ? pk + 128 * D : nullptr, (uint16_t*)p.dV + obase, 1.0f);
}

// D = rowsum(dO * O), read by both backward forms.  Coalesced: the LPR = d/8 lanes of
// a lane group read one row (16 bytes each: 16 lanes per 256-byte row at d = 128, 8
// per 128-byte row at d = 64), a wave 64/LPR rows per load and 32 rows in all, NL =
// 32 LPR / 64 loads of dO and of O in flight per lane.  Each lane sums its products
// in order, then the group adds its LPR partial sums by a butterfly (lane distance
// LPR/2 .. 1), which leaves every lane of the group the same total; lane i of the
// group keeps the total of its load i.
template <int D>
__global__ void __launch_bounds__(256) flash_bwd_delta_kernel(FbParams p) {
  constexpr int LPR = D / 8;           // lanes per row
  constexpr int RPL = 64 / LPR;        // rows per load
  constexpr int RPW = 32;              // rows per wave
  constexpr int NL = RPW / RPL;        // loads per lane
  static_assert(NL <= LPR, "a lane keeps at most one total");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPR, grp = lane / LPR;
  const int64_t rows = (int64_t)p.B * p.nH * p.T;
  const int64_t r0 = (int64_t)blockIdx.x * 128 + wave * RPW;  // first row of the wave
  u32x4_t gf[NL], of[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int64_t r = r0 + RPL * i + grp;  // row of [B, nH, T]
    if (r < rows) {
      const int64_t bh = r / p.T, t = r - bh * p.T;
      const int64_t b = bh / p.nH, h = bh - b * p.nH;
      const int64_t orow = p.o_bthd ? ((b * p.T + t) * p.nH + h) * D : (bh * p.T + t) * D;
      gf[i] = *(const u32x4_t*)((const __bf16*)p.dO + orow + 8 * sub);
      of[i] = *(const u32x4_t*)((const __bf16*)p.O + orow + 8 * sub);
    } else {
      gf[i] = of[i] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }
  float mine = 0.0f;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    float part = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2)
      part += bf16_bits_to_f32(gf[i][w2] & 0xffffu) * bf16_bits_to_f32(of[i][w2] & 0xffffu) +
              bf16_bits_to_f32(gf[i][w2] >> 16) * bf16_bits_to_f32(of[i][w2] >> 16);
#pragma unroll
    for (int m = LPR / 2; m >= 1; m >>= 1) part += __shfl_xor(part, m, 64);
    if (sub == i) mine = part;
  }
  const int64_t r = r0 + RPL * sub + grp;
  if (sub < NL && r < rows) p.delta[r] = mine;
}

// dK and dV of the key blocks the schedule cut into several units: the units'
// fp32 partials summed in unit order, dK scaled, both stored as bf16.  One thread
// per 4 consecutive d of one key.
template <int D>
__global__ void __launch_bounds__(256) flash_bwd_dkdv_reduce_kernel(FbParams p) {
  constexpr int QPK = D / 4;          // quads per key
  constexpr int PER = 128 * QPK;      // quads per key block
  const int BKV = p.B * p.nKV;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int i = (int)(gid / ((int64_t)BKV * PER));
  if (i >= p.n_split) return;
  const int rem = (int)(gid - (int64_t)i * BKV * PER);
  const int bkv = rem / PER, r = rem - (rem / PER) * PER;
  const int kl = r / QPK, d = (r - kl * QPK) * 4;
  const uint32_t sp = p.split[i];
  const int kbi = (int)(sp & 0xfffu), s0 = (int)((sp >> 12) & 0xfffu), ns = (int)(sp >> 24);
  const int key = kbi * 128 + kl;
  if (key >= p.T) return;
  f32x4_t ak = {0.f, 0.f, 0.f, 0.f}, av = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < ns; ++j) {
    const float* src = p.part + (((int64_t)bkv * p.n_slots + s0 + j) * 2 * 128 + kl) * D + d;
    ak += *(const f32x4_t*)src;
    av += *(const f32x4_t*)(src + 128 * D);
  }
  const int64_t o = ((int64_t)bkv * p.T + key) * D + d;
  *(u32x2_t*)((uint16_t*)p.dK + o) = u32x2_t{pack_bf16x2(ak[0] * p.scale, ak[1] * p.scale),
                                             pack_bf16x2(ak[2] * p.scale, ak[3] * p.scale)};
  *(u32x2_t*)((uint16_t*)p.dV + o) = u32x2_t{pack_bf16x2(av[0], av[1]), pack_bf16x2(av[2], av[3])};
}

// Balanced dK/dV schedule.  A key block's work is its iterations (query tiles of the
// group's heads); causal attention gives the first key blocks many more than the
// last, and one workgroup per key block leaves the CUs of the short ones idle while
// the long ones run (configuration 4: 64 iterations for key block 0, 8 for key block
// 7, 56 % of the CU time used).  Each key block is cut into units of at most W
// iterations and the units launch largest first, so the hardware's in-order dispatch
// to the CU that frees up first packs them (longest-processing-time-first).  A unit
// costs its iterations plus a fixed FB_UNIT_COST (the K/V load before its first tile,
// the halves' exchange and the dK/dV stores after its last; the dK/dV kernel holds a
// CU alone, so none of it overlaps another unit): W is the cut, from the even share
// W0 = total iterations / CUs up to 1.5 W0, whose simulated dispatch ends earliest
// (ties to the larger W: fewer partials to sum).  When the partials of the cut
// blocks do not fit the room given, W grows by half until they do; when the tables
// do not fit the kernel arguments, n_units stays 0.
constexpr int FB_UNIT_COST = 7;

// Unit lengths of a key block of `w` iterations cut at W: at most 8 units of
// max(W, ceil(w / 8)) iterations, the last one the remainder.
void cut_units(int w, int64_t W, std::vector<int>& out) {
  if (w <= W) {
    out.push_back(w);
    return;
  }
  const int c = (int)std::max<int64_t>(W, (w + 7) / 8);
  for (int j = 0; j * c < w; ++j) out.push_back(std::min(w, (j + 1) * c) - j * c);
}

// End of the busiest CU when the units (the same list for every one of the BKV
// (batch, KV head) pairs, largest first, dispatched unit-major as the kernel maps
// workgroups) go in order to the CU that frees up first, each costing its
// iterations + FB_UNIT_COST.
int64_t dkdv_makespan(std::vector<int> lens, int64_t BKV, int cus) {
  std::sort(lens.begin(), lens.end(), std::greater<int>());
  std::priority_queue<int64_t, std::vector<int64_t>, std::greater<int64_t>> free_at;
  for (int c = 0; c < cus; ++c) free_at.push(0);
  int64_t end = 0;
  for (const int len : lens)
    for (int64_t i = 0; i < BKV; ++i) {
      const int64_t t = free_at.top() + len + FB_UNIT_COST;
      free_at.pop();
      free_at.push(t);
      end = std::max(end, t);
    }
  return end;
}

void plan_dkdv_schedule(FbParams& p, int head_dim) {
  p.n_units = p.n_slots = p.n_split = 0;
  if (!p.dsT || !p.part || p.cus <= 0) return;
  const int NKB = p.k_blocks, nqt = (p.T + FA_BK - 1) / FA_BK;
  const int64_t BKV = (int64_t)p.B * p.nKV;
  const size_t slot_bytes = (size_t)BKV * 2 * 128 * (size_t)head_dim * sizeof(float);
  std::vector<int> w(NKB);
  int64_t sum = 0;
  for (int k = 0; k < NKB; ++k) {
    const int qt0 = p.causal ? k * 128 / FA_BK : 0;
    w[k] = nqt > qt0 ? (nqt - qt0) * p.group : 0;
    if (w[k] >= 65536) return;
    sum += w[k];
  }
  // The cut: simulated over W0 .. 1.5 W0 (configuration 4, W0 = 36: backward 171-173 us
  // at W = 36, 168-169 at 38, 167 at 39, 163-166 at 40, 166-170 at 42, 173-178 at 46;
  // the simulation picks 40).  The last choice is kept per thread for repeated calls.
  const int64_t W0 = std::max<int64_t>(1, (sum * BKV + p.cus - 1) / p.cus);
  struct CutCache { int64_t bkv, T, W; int nkb, group, causal, cus; };
  thread_local CutCache cache = {-1, -1, 0, 0, 0, 0, 0};
  int64_t Wbest = W0;
  if (cache.bkv == BKV && cache.T == p.T && cache.nkb == NKB && cache.group == p.group &&
      cache.causal == p.causal && cache.cus == p.cus) {
    Wbest = cache.W;
  } else {
    // at most 25 candidates, and no search when one simulation would dispatch over
    // 20 K workgroups (the host cost stays under a millisecond)
    const int64_t step = std::max<int64_t>(1, W0 / 48);
    int64_t best = -1;
    std::vector<int> lens;
    for (int64_t W = W0; W <= W0 + W0 / 2; W += step) {
      lens.clear();
      for (int k = 0; k < NKB; ++k) cut_units(w[k], W, lens);
      if ((int64_t)lens.size() * BKV > 20000) break;
      const int64_t m = dkdv_makespan(lens, BKV, p.cus);
      if (best < 0 || m <= best) {
        best = m;
        Wbest = W;
      }
    }
    cache = {BKV, p.T, Wbest, NKB, p.group, p.causal, p.cus};
  }
  struct Unit { int kbi, ib, ie, slot; };
  std::vector<Unit> units;
  int slots = 0, nsplit = 0;
  for (int64_t W = Wbest;; W += (W + 1) / 2) {
    units.clear();
    slots = nsplit = 0;
    bool fits = true;
    for (int k = 0; k < NKB && fits; ++k) {
      if (w[k] <= W) {
        units.push_back({k, 0, w[k], -1});
        continue;
      }
      const int c = (int)std::max<int64_t>(W, (w[k] + 7) / 8);  // at most 8 units
      const int n = (w[k] + c - 1) / c;
      if (nsplit >= FB_MAX_SPLIT || slots + n > 4095) return;
      p.split[nsplit++] = (uint32_t)k | (uint32_t)slots << 12 | (uint32_t)n << 24;
      for (int j = 0; j < n; ++j) units.push_back({k, j * c, std::min(w[k], (j + 1) * c), slots + j});
      slots += n;
      fits = (size_t)slots * slot_bytes <= p.part_bytes;
    }
    if (nsplit == 0) return;  // nothing to balance (or W outgrew every key block)
    if (fits) break;
  }
  if ((int)units.size() > FB_MAX_UNITS) return;
  std::stable_sort(units.begin(), units.end(),
                   [](const Unit& a, const Unit& b) { return a.ie - a.ib > b.ie - b.ib; });
  for (size_t u = 0; u < units.size(); ++u) {
    p.unit_kbi[u] = (uint32_t)units[u].kbi | (uint32_t)(units[u].slot + 1) << 16;
    p.unit_range[u] = (uint32_t)units[u].ib | (uint32_t)units[u].ie << 16;
  }
  p.n_units = (int)units.size();
  p.n_slots = slots;
  p.n_split = nsplit;
}

}  // namespace

int flash_fwd_blocks(int T) { return (T + FA_BQ - 1) / FA_BQ; }

size_t flash_bwd_partial_bytes(int64_t B, int64_t nH, int64_t T) {
  return (size_t)B * (size_t)nH * (size_t)T * 128 * sizeof(float);
}

template <int D>
hipError_t launch_flash_bwd_d(FbParams& p, hipStream_t stream) {
  plan_dkdv_schedule(p, D);
  // D first (both kernels after it read it); then, without the dS^T workspace, the dQ
  // kernel.  With it the dK/dV kernel writes dS^T and the caller runs dQ = scale * dS K.
  const int64_t rows = (int64_t)p.B * p.nH * p.T;
  hipLaunchKernelGGL(flash_bwd_delta_kernel<D>, dim3((unsigned)((rows + 127) / 128)), dim3(256), 0,
                     stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (!p.dsT) {
    const int64_t nq = (int64_t)p.B * p.nH * p.q_blocks;
    hipLaunchKernelGGL(flash_bwd_dq_kernel<D>, dim3((unsigned)nq), dim3(256), 0, stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const int64_t nk = (int64_t)p.B * p.nKV * (p.n_units ? p.n_units : p.k_blocks);
  if (p.dsT)
    hipLaunchKernelGGL((flash_bwd_dkdv_kernel<D, true>), dim3((unsigned)nk), dim3(512), 0, stream, p);
  else
    hipLaunchKernelGGL((flash_bwd_dkdv_kernel<D, false>), dim3((unsigned)nk), dim3(512), 0, stream, p);
  if (!p.n_split) return hipGetLastError();
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t quads = (int64_t)p.n_split * p.B * p.nKV * 128 * (D / 4);
  hipLaunchKernelGGL(flash_bwd_dkdv_reduce_kernel<D>, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0,
                     stream, p);
  return hipGetLastError();
}

hipError_t launch_flash_bwd(const FbParams& p_in, int head_dim, hipStream_t stream) {
  FbParams p = p_in;
  if (head_dim == 128) return launch_flash_bwd_d<128>(p, stream);
  if (head_dim == 64) return launch_flash_bwd_d<64>(p, stream);
  return hipErrorInvalidValue;
}

int flash_bwd_key_blocks(int T) { return (T + 127) / 128; }

hipError_t launch_flash_fwd(const FaParams& p, int head_dim, hipStream_t stream) {
  const int64_t n = (int64_t)p.B * p.nH * p.q_blocks;
  if (head_dim == 128)
    hipLaunchKernelGGL(flash_fwd_kernel<128>, dim3((unsigned)n), dim3(256), 0, stream, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(flash_fwd_kernel<64>, dim3((unsigned)n), dim3(256), 0, stream, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace mig
