// mi_gemm_dlds.hpp -- bf16 and fp32 GEMM main loop with direct-to-LDS loads (gfx950).
//
// Operand tiles move global -> LDS with buffer_load_dwordx4 ... lds: each lane's
// 16 bytes land at M0 + 16*lane, so the LDS layout (and its bank swizzle) is set
// by which global chunk each lane fetches.  No staging registers, no LDS store
// instructions and no register transposes are involved, which frees the VGPRs
// for a STAGES-deep ring of LDS tiles.
//
// The main loop is unrolled by STAGES so every LDS address is a per-lane base
// register plus an immediate offset, and every DMA is one buffer load whose
// per-lane offset never changes: the K position of a tile lives in the buffer
// descriptor (base moved to the tile, extent shrunk by the same amount, so the
// hardware bounds check still zero-fills everything outside the matrix) and M0
// comes from scalar registers.  With one wave per SIMD the wave must issue
// every MFMA itself; address arithmetic between them is issue time the MFMA
// pipe loses.
//
// LDS layouts (one region per operand, STAGES stage buffers per region):
//   K-contiguous operand  [R rows][BK]  (NCH = BK/8 chunks of 16 bytes per row,
//       chunk position XOR-swizzled by the row); MFMA fragments are ds_read_b128.
//   row-contiguous operand [BK k-rows][R]  (R/8 chunks per k-row, chunk index
//       XOR-swizzled by the k-row); MFMA fragments are two ds_read_b64_tr_b16,
//       whose 16-lane groups turn a 4 (k) x 16 (row) block into 16 lanes x 4 k.
//       fp32: four ds_read_b32 per fragment (mc_swz32).
// The read patterns are bank-conflict free on the 64-bank LDS.
#pragma once
#include "mi_gemm_device.hpp"

namespace mig {

typedef __attribute__((address_space(3))) u32x4_t lds_u32x4_t;

#define MIG_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// s_waitcnt vmcnt(N) with expcnt and lgkmcnt left unconstrained (gfx9 encoding:
// vmcnt[3:0] bits 3:0, vmcnt[5:4] bits 15:14, expcnt bits 6:4, lgkmcnt bits 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier for the LDS ring: this wave's LDS reads and writes are
// complete (lgkmcnt(0)) but its DMA loads may still be in flight -- the caller
// waits for the ones it needs with wait_vmcnt first.  (__syncthreads() would
// also wait for every outstanding DMA load, emptying the ring.)  The empty asm
// statements keep the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_ring_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt(63), expcnt(7) = no constraint
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Chunk position of K-chunk c in row r of a K-contiguous tile with NCH chunks
// per row.  16 consecutive rows read at one c hit 16 distinct 16-byte bank
// groups of the 64-bank LDS (rows of 64 or 128 bytes).
template <int NCH>
__device__ __forceinline__ int kc_swz(int r, int c) {
  if constexpr (NCH == 4) return c ^ ((r >> 2) & 3);
  else return c ^ ((r ^ (r >> 3)) & 7);
}

// Physical chunk of logical chunk q in k-row kr of a row-contiguous tile with
// CPR chunks per k-row (CPR a power of two >= 16): the four k-rows one transpose
// read touches land in four different 64-byte bank groups.
template <int CPR>
__device__ __forceinline__ int mc_swz(int kr, int q) {
  static_assert((CPR & (CPR - 1)) == 0 && CPR >= 16, "XOR swizzle needs 2^n >= 16 chunks per k-row");
  return q ^ ((kr & 3) << 2);
}
// Inverse of mc_swz: the logical chunk stored at position p of k-row kr.
template <int CPR>
__device__ __forceinline__ int mc_unswz(int kr, int p) {
  return p ^ ((kr & 3) << 2);
}

// fp32 row-contiguous tiles: chunk q of k-row kr sits at q ^ 8 on k-rows 4..7 (mod
// 8).  A fragment read takes 32 consecutive columns (8 chunks, 128 bytes) of k-row
// kr in lanes 0-31 and of k-row kr + 4 in lanes 32-63: the two halves of the
// 256-byte bank window.  Self-inverse.
__device__ __forceinline__ int mc_swz32(int kr, int q) { return q ^ (((kr >> 2) & 1) << 3); }

// Row-contiguous tiles whose row is not a power of two (192 columns) are stored
// in 128-byte granules, column block by column block: granule G holds k-row
// G % BK of the 64-column block G / BK, so consecutive k-rows of one column block
// are 128 bytes apart and any four of them cover both halves of a 256-byte bank
// window; the two 64-byte halves of a granule swap on k-rows 2 and 3 (mod 4), so
// the four k-rows one transpose read touches land in four different 64-byte bank
// groups.  A k-row of R columns would instead start at R * 2 bytes (384: an odd
// multiple of 128), and no chunk rotation of it avoids two k-rows meeting in one
// bank group for every 32-column block.
__device__ __forceinline__ int gran_half(int kr) { return ((kr >> 1) & 1) << 6; }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)MIG_LDS_PTR(p);
}

// Buffer descriptor from values the caller keeps in scalar registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t scalar_rsrc(const void* base, uint32_t ext) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)ext, kBufFlags);
}

#ifndef MI_DLDS_EARLY
#define MI_DLDS_EARLY 1
#endif

template <int I>
using ic = std::integral_constant<int, I>;

template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(ic<I>{});
    static_for<N, I + 1>(f);
  }
}

// One operand of the direct-to-LDS pipeline.  R: tile rows (M or N extent),
// BK: K extent of a stage (elements), KC: K-contiguous in memory, WT: rows of the
// wave tile (fragments of 32 rows each), NW: waves sharing the DMA, NSUBW: K
// substeps one wave computes per stage (all of them, or half when two wave groups
// split each stage's K range), ES: element bytes (2: bf16, 4: fp32).  A substep
// covers 32 bytes of every row: 16 bf16 (one 32x32x16 MFMA) or 8 fp32 (four
// 32x32x2 MFMAs).
template <int R, int BK, bool KC, int STAGES, int WT, int NW = 4, int NSUBW = BK / 16, int ES = 2>
struct DldsOperand {
  static constexpr int EPC = 16 / ES;                 // elements per 16-byte chunk
  static constexpr int NCH = BK / EPC;                // KC: 16-byte chunks per row
  static constexpr int CPR = R / EPC;                 // !KC: 16-byte chunks per k-row
  static constexpr bool GRAN = !KC && (CPR & (CPR - 1)) != 0;  // 128-byte granule layout
  static constexpr int KRB = GRAN ? 128 : R * ES;     // !KC: LDS bytes between k-rows
  static_assert(!GRAN || R % 64 == 0, "granule layout needs 64-column blocks");
  static_assert(ES == 2 || (!GRAN && (KC || CPR >= 16)), "fp32 k-rows: 2^n >= 16 chunks");
  static constexpr int BYTES = R * BK * ES;           // one stage of this operand
  static constexpr int NBLK = BYTES / 1024;           // 1 KB DMA blocks per stage
  static constexpr int NU = NBLK / NW;                // DMA instructions per wave
  static constexpr int NSUB = BK * ES / 32;
  static constexpr int NF = WT / 32;                  // fragments per wave
  static constexpr int NRB = KC ? 2 * NSUBW : NF;     // read base registers
  static_assert(BYTES % 1024 == 0 && NBLK % NW == 0, "tile must split into whole DMA blocks per wave");
  static_assert(NSUB % NSUBW == 0, "wave groups split the stage's substeps evenly");
  // largest immediate offset added to a read base must fit the 16-bit DS offset
  static constexpr int MAX_IMM = KC ? ((NF - 1) / 2) * 64 * BK * ES + (STAGES - 1) * BYTES
                                 : ES == 2 ? (16 * (NSUBW - 1) + 4) * KRB + (STAGES - 1) * BYTES
                                           : (8 * (NSUBW - 1) + 3) * KRB + (STAGES - 1) * BYTES;
  static_assert(MAX_IMM < 65536, "LDS read offsets exceed the DS immediate");

  uint32_t voff[NU];  // byte offset of unit u from the tile's first K (kBufOOB: row outside)
  int klim[NU];       // KC: the unit's chunk is inside the K extent while k0 < klim[u]
  uint32_t rb[NRB];   // LDS address of fragment reads, stage 0
  uint32_t dma;       // wave-uniform LDS address of this wave's first DMA block, stage 0

  // DMA offsets.  ld: leading dimension (elements), rows: M or N extent, row0:
  // first tile row, kseg: K extent of a segment.
  __device__ __forceinline__ void init_dma(int64_t ld, int rows, int row0, int kseg) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ldb = (int)ld * ES;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int b = wave * NU + u;
      if constexpr (KC) {
        const int row = b * (64 / NCH) + lane / NCH;
        const int c = kc_swz<NCH>(row, lane % NCH);
        voff[u] = (uint32_t)((row0 + row) * ldb + c * 16);  // rows >= M lie past the extent
        klim[u] = kseg - c * EPC;
      } else if constexpr (GRAN) {
        // LDS chunk qi: granule qi / 8 = k-row kr of 64-column block qi / 8 / BK
        const int qi = b * 64 + lane;
        const int gi = qi >> 3, kr = gi % BK;
        const int col = (gi / BK) * 64 + (((qi & 7) * 16) ^ gran_half(kr)) / 2;
        const int grow = row0 + col;
        voff[u] = grow < rows ? (uint32_t)(kr * ldb + grow * 2) : kBufOOB;
        klim[u] = 0;
      } else {
        // chunk q of the stage lands at LDS chunk q: k-row q / CPR, position q % CPR
        const int qi = b * 64 + lane;
        const int kr = qi / CPR;
        const int q = ES == 2 ? mc_unswz<CPR>(kr, qi - kr * CPR) : mc_swz32(kr, qi - kr * CPR);
        const int grow = row0 + q * EPC;
        voff[u] = grow < rows ? (uint32_t)(kr * ldb + grow * ES) : kBufOOB;
        klim[u] = 0;
      }
    }
  }

  // LDS addresses.  region: LDS address of this operand's stage 0; w0: first row
  // of the wave tile; wave_u: wave index (among the NW) held in a scalar
  // register; ks0: first of the NSUBW substeps this wave reads.
  __device__ __forceinline__ void init_lds(uint32_t region, int w0, int wave_u, int ks0 = 0) {
    const int lane = threadIdx.x & 63;
    dma = region + (uint32_t)(wave_u * NU * 1024);
    if constexpr (KC) {
#pragma unroll
      for (int s = 0; s < NSUBW; ++s)
#pragma unroll
        for (int par = 0; par < 2; ++par) {
          const int r = w0 + 32 * par + (lane & 31);
          const int c = 2 * (ks0 + s) + (lane >> 5);
          rb[2 * s + par] = region + (uint32_t)(r * (BK * ES) + 16 * kc_swz<NCH>(r, c));
        }
    } else if constexpr (ES == 4) {
      // lane: column n of fragment f, k-rows 4h .. 4h+3 of each 8-k substep (h = lane / 32)
      const int h = lane >> 5;
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const int n = w0 + 32 * f + (lane & 31);
        const int kr = 8 * ks0 + 4 * h;
        rb[f] = region + (uint32_t)(kr * KRB + 16 * mc_swz32(kr, n >> 2) + 4 * (n & 3));
      }
    } else {
      const int g = lane >> 4, j = lane & 15;
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const int col = w0 + 32 * f + (g & 1) * 16 + 4 * (j & 3);
        const int q = col >> 3, sub = (col & 7) * 2;
        const int krb = 8 * (g >> 1) + (j >> 2);
        if constexpr (GRAN)
          rb[f] = region + (uint32_t)(((col >> 6) * BK + krb + 16 * ks0) * 128 +
                                      (((col & 63) * 2) ^ gran_half(krb)));
        else
          rb[f] = region + (uint32_t)((krb + 16 * ks0) * (R * 2) + 16 * mc_swz<CPR>(krb, q) + sub);
      }
    }
  }

  // DMA unit u of the K tile at element offset k0 (descriptor `rs` already
  // positioned at that tile) into stage J of the region whose wave base is `dst`.
  template <int J, bool KTAIL>
  __device__ __forceinline__ void load(int u, __amdgpu_buffer_rsrc_t rs, int k0, uint32_t dst) const {
    uint32_t vo = voff[u];
    if constexpr (KC && KTAIL) vo = (k0 < klim[u]) ? vo : kBufOOB;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rs, (__attribute__((address_space(3))) void*)(uintptr_t)(dst + (uint32_t)(J * BYTES + u * 1024)),
        16, (int)vo, 0, 0, 0);
  }

  // MFMA fragment f (rows w0+32f .. +31 of the wave tile), K substep S of stage J,
  // as 8 bf16 per lane.  In a K-contiguous tile fragments f and f+2 share the
  // swizzle, 64 rows apart; a row-contiguous tile steps 16 k-rows per substep.
  template <int S, int J>
  __device__ __forceinline__ u32x4_t frag(int f) const {
    if constexpr (KC) {
      const uint32_t a = rb[2 * S + (f & 1)] + (uint32_t)((f >> 1) * 64 * BK * ES + J * BYTES);
      return *(const lds_u32x4_t*)(uintptr_t)a;
    } else if constexpr (ES == 4) {
      // fp32 k-rows 8S + 4h + t, t = 0..3: value t feeds the substep's MFMA t
      typedef __attribute__((address_space(3))) const uint32_t lds_u32_t;
      u32x4_t out;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        out[t] = *(lds_u32_t*)(uintptr_t)(rb[f] + (uint32_t)((8 * S + t) * KRB + J * BYTES));
      return out;
    } else {
      u32x4_t out = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        u32x2_t w = {0u, 0u};
#if defined(__HIP_DEVICE_COMPILE__)
        // Issued as inline asm: the compiler makes the transpose-read builtin wait
        // for every LDS-DMA load in flight (vmcnt(0)), which would drain the ring.
        // The result is pending until the substep-start lgkmcnt(0) wait that
        // precedes its first use (see substep()).
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                     : "=v"(w)
                     : "v"(rb[f]), "i"((16 * S + 4 * t) * KRB + J * BYTES));
#endif
        out[2 * t] = w[0];
        out[2 * t + 1] = w[1];
      }
      return out;
    }
  }
};

// Kernel variants (VAR bits): the K segment length is not a multiple of BK
// (K-contiguous operands then mask the chunks past the segment end), and the
// problem takes the direct epilogue (every tile full, epilogue alpha / SiLU
// gate, beta*C and the output conversion only, no split-K).  One kernel holding
// both epilogues would need the accumulators in two places at once.
enum { DLDS_KTAIL = 1, DLDS_FAST_EPI = 2, DLDS_ROWSCALE = 4 };

// GEMM of WGM x WGN waves, wave tile (BM/WGM) x (BN/WGN) of 32x32 MFMA blocks: bf16
// (ES = 2, one 32x32x16 MFMA per block and substep) or fp32 (ES = 4, four 32x32x2).
// KG = 2 (wave-level split-K): a second group of WGM x WGN waves computes the
// same output tile over the other half of every LDS stage's K range (both
// groups share the stage's DMA), so a workgroup keeps two waves per SIMD on one
// output tile; the groups' accumulators are summed through LDS before the
// epilogue, each group then storing half of the tile.
template <int BM, int BN, int BK, int STAGES, bool AK, bool BKC, int MODE, int VAR, int WGM = 2,
          int WGN = 2, int KG = 1, int ES = 2>
__global__ void __launch_bounds__(64 * WGM * WGN * KG)
    __attribute__((amdgpu_waves_per_eu(WGM * WGN * KG / 4)))
    gemm_dlds_kernel(Params p) {
  constexpr bool KTAIL = (VAR & DLDS_KTAIL) != 0;
  constexpr bool FAST_EPI = (VAR & DLDS_FAST_EPI) != 0;
  // ROWSCALE: the direct epilogue multiplies row m by p.row_scale[m] (a folded RMSNorm);
  // a variant of its own, so that the plain GEMMs carry no row-scale code (+0.45 % on the
  // configuration-3 set, one box)
  constexpr bool ROWSCALE = (VAR & DLDS_ROWSCALE) != 0;
  constexpr int NWG = WGM * WGN;          // waves of one K group
  constexpr int NWAVE = NWG * KG;         // waves of the workgroup
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr bool DUAL = (MODE == MODE_DUAL);
  constexpr int NB = DUAL ? 2 * TN : TN;
  constexpr int NSUBT = BK * ES / 32;     // K substeps of a stage (32 bytes of every row)
  constexpr int NSUB = NSUBT / KG;        // K substeps one wave computes per stage
  static_assert(MODE != MODE_PROLOGUE, "the SiLU-gate prologue needs register staging");
  static_assert(KG == 1 || KG == 2, "one or two K groups");
  static_assert(KG == 1 || (MODE == MODE_PLAIN && TM == 2), "split-K groups: plain mode, two row blocks");
  static_assert(NSUB == 2 || NSUB == 4, "each wave computes 2 or 4 substeps per stage");
  static_assert(STAGES >= 2 && STAGES <= 4, "2..4 stages");
  static_assert(ES == 2 || (ES == 4 && !DUAL), "bf16, or fp32 without the dual B");
  // TRR: fragments of a row-contiguous bf16 operand come from transpose reads issued
  // as inline asm, whose completion the code waits for itself
  constexpr bool TRR = ES == 2 && (!AK || !BKC);
  using OpA = DldsOperand<BM, BK, AK, STAGES, WTM, NWAVE, NSUB, ES>;
  using OpB = DldsOperand<BN, BK, BKC, STAGES, WTN, NWAVE, NSUB, ES>;
  constexpr int A_REG = 0;                                   // LDS regions (bytes)
  constexpr int B_REG = A_REG + STAGES * OpA::BYTES;
  constexpr int B2_REG = B_REG + STAGES * OpB::BYTES;
  constexpr int LDS_BYTES = B2_REG + (DUAL ? STAGES * OpB::BYTES : 0);
  constexpr int NL = OpA::NU + OpB::NU * (DUAL ? 2 : 1);    // DMA instructions per wave per tile
  static_assert(NL * STAGES < 64, "vmcnt range");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS ring exceeds 160 KB");

  __shared__ __attribute__((aligned(16))) char smem[LDS_BYTES];
  const uint32_t lds0 = lds_addr(smem);

  const int nblocks = gridDim.x;
  const TileCoord tc = map_tile(blockIdx.x, nblocks, p.tiles_m, p.tiles_n, p.splits, p.causal, p.group_m);
  const int m0 = uniform(tc.tm * BM), n0 = uniform(tc.tn * BN);
  const int zo = uniform(tc.z / p.heads), zi = uniform(tc.z - (tc.z / p.heads) * p.heads);
  const int ziA = uniform(zi / p.gA), ziB = uniform(zi / p.gB), ziC = uniform(zi / p.gC);
  const char* Ab = uniform((const char*)p.A + ((int64_t)zo * p.aO + (int64_t)ziA * p.aI) * ES);
  const char* Bb = uniform((const char*)p.B + ((int64_t)zo * p.bO + (int64_t)ziB * p.bI) * ES);
  const char* B2b = DUAL ? uniform((const char*)p.B2 + ((int64_t)zo * p.bO + (int64_t)ziB * p.bI) * ES)
                         : nullptr;
  const int64_t coff = (int64_t)zo * p.cO + (int64_t)ziC * p.cI;
  void* Cz = (char*)p.C + coff * (p.c_bf16 ? 2 : 4);
  const void* Rz = p.R ? (const char*)p.R + ((int64_t)zo * p.rO + (int64_t)zi * p.rI) * (p.r_bf16 ? 2 : 4)
                       : nullptr;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wave_u = uniform(wave);
  const int kg = uniform(wave / NWG);     // K group
  const int wq = wave % NWG;              // wave within the group
  const int wm = wq / WGN, wn = wq % WGN;

  if (p.causal == CAUSAL_OUT_LOWER && n0 > m0 + BM - 1) {
    if (p.splits > 1) return;  // the reduction kernel writes the mask
    for (int idx = threadIdx.x; idx < BM * BN; idx += 64 * NWAVE) {
      const int m = m0 + idx / BN, n = n0 + idx % BN;
      if (m < p.M && n < p.N) {
        const int64_t ci = (int64_t)m * p.ldc + n;
        if (p.c_bf16)
          ((uint16_t*)Cz)[ci] = (uint16_t)f32_to_bf16_rne(p.mask_value);
        else
          ((float*)Cz)[ci] = p.mask_value;
      }
    }
    return;
  }

  const int kt_seg = (p.K + BK - 1) / BK;
  int klo = 0, khi = kt_seg;
  if (p.causal == CAUSAL_A_LOWER) {
    const int lim = (m0 + BM + BK - 1) / BK;
    khi = khi < lim ? khi : lim;
  } else if (p.causal == CAUSAL_A_UPPER) {
    klo = m0 / BK;
  }
  klo = uniform(klo);
  const int per_seg = uniform(khi > klo ? khi - klo : 0);
  const int total = per_seg * p.nseg;
  const int it0 = uniform((int)((int64_t)total * tc.split / p.splits));
  const int it1 = uniform((int)((int64_t)total * (tc.split + 1) / p.splits));

  f32x16_t acc[TM][NB];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  OpA oa;
  OpB ob;
  OpB ob2;  // DUAL: LDS addresses of the second B (DMA offsets shared with ob)
  oa.init_dma(p.lda, p.M, m0, p.K);
  ob.init_dma(p.ldb, p.N, n0, p.K);
  oa.init_lds(lds0 + A_REG, wm * WTM, wave_u, kg * NSUB);
  ob.init_lds(lds0 + B_REG, wn * WTN, wave_u, kg * NSUB);
  if constexpr (DUAL) ob2.init_lds(lds0 + B2_REG, wn * WTN, wave_u);

  // Tile stream of the DMA.  Descriptors start at the tile (base + K offset,
  // extent reduced by the same amount) and step by one K tile; crossing into
  // the next K segment re-seats them at that segment's first tile.  A tile past
  // it1 gets an empty extent and loads zeros.
  const uint32_t a_step = (uint32_t)BK * (AK ? (uint32_t)ES : (uint32_t)p.lda * ES);  // bytes per K tile
  const uint32_t b_step = (uint32_t)BK * (BKC ? (uint32_t)ES : (uint32_t)p.ldb * ES);
  // K rotation (krot; one problem, one K segment, no split, no causal skipping):
  // the workgroups of XCD x (hardware dispatch: block id mod 8) walk the K tiles
  // starting at tile x*per_seg/8 and wrap around (the segment-crossing step below
  // re-seats the descriptors at the same matrix, segA and segB being 0).  All tiles
  // of one XCD still share their A and B panels in its L2 at the same K, but the
  // eight XCDs read different rows of the operands at any moment, so the first
  // XCD to touch a row takes the HBM latency and the others find it in the
  // memory-side last-level cache, instead of all eight missing on the same rows
  // together.  The order of the fp32 sum over K tiles changes with the XCD index
  // and is fixed for a given problem and plan.
  const int rot = p.krot ? uniform((int)(((int64_t)(blockIdx.x & 7) * per_seg) >> 3)) : 0;
  int d_it = it0;
  int d_seg = uniform(per_seg > 0 ? it0 / per_seg : 0);
  int d_kt = uniform(it0 - d_seg * per_seg + rot);
  const char* a_ptr = Ab + (int64_t)d_seg * p.segA * ES + (uint32_t)(klo + d_kt) * a_step;
  const char* b_ptr = Bb + (int64_t)d_seg * p.segB * ES + (uint32_t)(klo + d_kt) * b_step;
  const char* b2_ptr = DUAL ? B2b + (int64_t)d_seg * p.segB * ES + (uint32_t)(klo + d_kt) * b_step
                            : nullptr;
  uint32_t a_ext = p.extA - (uint32_t)(klo + d_kt) * a_step;
  uint32_t b_ext = p.extB - (uint32_t)(klo + d_kt) * b_step;
  struct TileRef {
    __amdgpu_buffer_rsrc_t ra, rb, rb2;
    int k0;
  };
  auto next_tile = [&]() __attribute__((always_inline)) {
    TileRef t;
    const bool live = d_it < it1;
    t.k0 = (klo + d_kt) * BK;
    t.ra = scalar_rsrc(a_ptr, live ? a_ext : 0u);
    t.rb = scalar_rsrc(b_ptr, live ? b_ext : 0u);
    if constexpr (DUAL) t.rb2 = scalar_rsrc(b2_ptr, live ? b_ext : 0u);
    ++d_it;
    a_ptr += a_step;
    b_ptr += b_step;
    if constexpr (DUAL) b2_ptr += b_step;
    a_ext -= a_step;
    b_ext -= b_step;
    if (++d_kt == per_seg) {  // next K segment
      d_kt = 0;
      a_ptr += (int64_t)p.segA * ES - (int64_t)per_seg * a_step;
      b_ptr += (int64_t)p.segB * ES - (int64_t)per_seg * b_step;
      if constexpr (DUAL) b2_ptr += (int64_t)p.segB * ES - (int64_t)per_seg * b_step;
      a_ext += per_seg * a_step;
      b_ext += per_seg * b_step;
    }
    return t;
  };
  constexpr bool KTA = KTAIL && AK, KTB = KTAIL && BKC;
  auto dma = [&](int o, const TileRef& t, auto JF_c) __attribute__((always_inline)) {
    constexpr int JF = decltype(JF_c)::value;
    if (o < OpA::NU) oa.template load<JF, KTA>(o, t.ra, t.k0, oa.dma);
    else if (o < OpA::NU + OpB::NU) ob.template load<JF, KTB>(o - OpA::NU, t.rb, t.k0, ob.dma);
    else ob.template load<JF, KTB>(o - OpA::NU - OpB::NU, t.rb2, t.k0, ob2.dma);
  };

  // EARLY (two stages of four substeps): each substep has its own fragment set,
  // so a K tile's fragments are all read by the end of its second substep and
  // its stage is free from then on; otherwise substep s uses set s & 1.
  constexpr bool EARLY = MI_DLDS_EARLY && STAGES == 2 && NSUB == 4;
  constexpr int NSET = EARLY ? 4 : 2;
  u32x4_t fa[NSET][TM], fb[NSET][NB];
  constexpr int NREAD = TM + NB;  // fragments per substep
  auto read_op = [&](int o, auto JR_c, auto S_c, int set) __attribute__((always_inline)) {
    constexpr int JR = decltype(JR_c)::value, S = decltype(S_c)::value;
    if (o < TM) {
      fa[set][o] = oa.template frag<S, JR>(o);
    } else {
      const int j = o - TM;
      if (DUAL && j >= TN) fb[set][j] = ob2.template frag<S, JR>(j - TN);
      else fb[set][j] = ob.template frag<S, JR>(j);
    }
  };
  auto mfma_op = [&](int set, int i, int j) __attribute__((always_inline)) {
    if constexpr (ES == 2) {
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, fb[set][j]),
                                                          __builtin_bit_cast(bf16x8_t, fa[set][i]),
                                                          acc[i][j], 0, 0, 0);
    } else {
      // fp32: value t of both fragments is k = 8S + t (lanes 0-31) and 8S + 4 + t
      // (lanes 32-63), the two k of one 32x32x2 MFMA
#pragma unroll
      for (int t = 0; t < 4; ++t)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(fb[set][j][t]),
                                                         __uint_as_float(fa[set][i][t]), acc[i][j], 0, 0, 0);
    }
  };

  // One substep = TM*NB MFMA slots.  The fragment reads of the next substep go
  // out one per slot from the first slot on, so they have most of the substep
  // to land before its lgkmcnt wait.  DMA instructions are spread over MFMA
  // slots: a wave that issues them faster than the memory pipeline accepts
  // them stalls in order, and the MFMAs behind them with it.  With three or
  // more stages (SPREAD) the DMA of the K tile STAGES-1 ahead goes into the
  // stage freed at the previous barrier and is spread over every slot of the
  // K tile; with two stages it can only start after this tile's barrier and is
  // spread over the last substep.  A scheduling fence after every slot keeps
  // that order.
  constexpr int NS = TM * NB;
  constexpr int TOT = NSUB * NS;  // MFMA slots per K tile
  constexpr bool SPREAD = STAGES >= 3;
  // SPREAD: DMA instructions issued before the last substep of a K tile.
  constexpr int DMA_EARLY = (NL * (NSUB - 1) * NS + TOT - 1) / TOT;
  // at most one fragment read per MFMA slot (an fp32 slot is four MFMAs and may take more)
  static_assert(NREAD <= NS || ES == 4, "one fragment read per MFMA slot at most");
  // fragment reads of slot q: one each in the first NREAD slots, or spread evenly
  auto slot_reads = [&](int q, auto JR_c, auto RS_c, int set) __attribute__((always_inline)) {
    if constexpr (NREAD <= NS) {
      if (q < NREAD) read_op(q, JR_c, RS_c, set);
    } else {
#pragma unroll
      for (int o = (q * NREAD + NS - 1) / NS; o < ((q + 1) * NREAD + NS - 1) / NS; ++o)
        read_op(o, JR_c, RS_c, set);
    }
  };
  // S: substep index within the tile (fragment set S & 1).  RS / JR: substep
  // and stage whose fragments are read into the other set.  DMA: 0 none, 1 the
  // whole DMA of tile t spread over this substep, 2 the share of slots
  // S*NS .. S*NS+NS-1 of a DMA spread over the K tile.  JF: DMA stage.
  auto substep = [&](auto S_c, auto RS_c, auto JR_c, auto DMA_c, auto JF_c, const TileRef& t)
                     __attribute__((always_inline)) {
    constexpr int S = decltype(S_c)::value;
    constexpr int DMA = decltype(DMA_c)::value;
    constexpr int set = S & 1;
    if constexpr (TRR) {
      // fragments of this set issued by transpose-read asm are complete only
      // after lgkmcnt(0); nothing may be scheduled above this point
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      mfma_op(set, q / NB, q % NB);
      slot_reads(q, JR_c, RS_c, set ^ 1);
      if constexpr (DMA == 1) {
#pragma unroll
        for (int o = (q * NL + NS - 1) / NS; o < ((q + 1) * NL + NS - 1) / NS; ++o) dma(o, t, JF_c);
      } else if constexpr (DMA == 2) {
        const int g = S * NS + q;
#pragma unroll
        for (int o = (g * NL + TOT - 1) / TOT; o < ((g + 1) * NL + TOT - 1) / TOT; ++o) dma(o, t, JF_c);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // LDS instructions that read one fragment set (transpose reads take two per
  // fragment); the lgkmcnt field holds at most 15.
  constexpr int READ_OPS = TM * (AK ? 1 : 2) + NB * (BKC ? 1 : 2);
  constexpr int LGKM_KEEP = READ_OPS < 15 ? READ_OPS : 15;
  // EARLY substep S computes with set S, reads set RSET (substep RS of the
  // tile in stage JR) one fragment per slot, and issues half DPART (1 or 2; 0
  // none) of the DMA of tile t into stage JF spread over its slots.
  auto substep4 = [&](auto S_c, auto RSET_c, auto RS_c, auto JR_c, auto DPART_c, auto JF_c,
                      const TileRef& t) __attribute__((always_inline)) {
    constexpr int S = decltype(S_c)::value, RSET = decltype(RSET_c)::value;
    constexpr int DPART = decltype(DPART_c)::value;
    // first half NL/2 instructions, second half the rest (NL may be odd)
    constexpr int H0 = DPART == 2 ? NL / 2 : 0;
    constexpr int HN = DPART == 1 ? NL / 2 : DPART == 2 ? NL - NL / 2 : 0;
    if constexpr (TRR) {
      // set S was read two substeps ago; the previous substep's LDS reads (one
      // set, READ_OPS instructions) may stay in flight: LDS returns in order
      __builtin_amdgcn_s_waitcnt(0xC07F | (LGKM_KEEP << 8));
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      mfma_op(S, q / NB, q % NB);
      slot_reads(q, JR_c, RS_c, RSET);
#pragma unroll
      for (int o = H0 + (q * HN + NS - 1) / NS; o < H0 + ((q + 1) * HN + NS - 1) / NS; ++o)
        dma(o, t, JF_c);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Prologue: K tiles it0 .. it0+PRE-1 into stages 0 .. PRE-1.
  constexpr int PRE = SPREAD ? STAGES - 1 : STAGES;
  if (it0 < it1) {
    static_for<PRE>([&](auto J_c) __attribute__((always_inline)) {
      const TileRef t = next_tile();
#pragma unroll
      for (int o = 0; o < NL; ++o) dma(o, t, J_c);
    });
    wait_vmcnt<NL * (PRE - 1)>();
  }
  lds_ring_barrier();
  if (it0 < it1) {
#pragma unroll
    for (int o = 0; o < NREAD; ++o) read_op(o, ic<0>{}, ic<0>{}, 0);
    if constexpr (EARLY) {
#pragma unroll
      for (int o = 0; o < NREAD; ++o) read_op(o, ic<0>{}, ic<1>{}, 1);
    }
  }

  // K tile `it` sits in stage J = (it - it0) mod STAGES: substeps 0 .. NSUB-2
  // read stage J, then -- once this wave's DMA of tile it+1 has landed -- a
  // barrier after which no wave reads stage J again, then the last substep runs
  // while reading substep 0 of tile it+1.
  //   SPREAD: every substep also issues its share of the DMA of tile
  //   it+STAGES-1 into the stage of tile it-1 (free since the previous
  //   barrier).  At the wait, the DMAs younger than tile it+1 are the STAGES-3
  //   tiles after it and the DMA_EARLY instructions of this tile's share.
  //   Two stages: the last substep issues the DMA of tile it+2 into stage J.
  // The loop runs in whole rounds of STAGES tiles; tiles past it1 are all-zero
  // (empty descriptors) and add nothing.
  using DmaMode = ic<SPREAD ? 2 : 0>;
  using DmaLast = ic<SPREAD ? 2 : 1>;
  constexpr int VM_WAIT = SPREAD ? NL * (STAGES - 3) + DMA_EARLY : 0;
  auto iteration = [&](auto J_c) __attribute__((always_inline)) {
    constexpr int J = decltype(J_c)::value;
    constexpr int JN = (J + 1) % STAGES;
    constexpr int JF = SPREAD ? (J + STAGES - 1) % STAGES : J;
    const TileRef t = next_tile();
    substep(ic<0>{}, ic<1>{}, ic<J>{}, DmaMode{}, ic<JF>{}, t);
    if constexpr (NSUB == 4) {
      substep(ic<1>{}, ic<2>{}, ic<J>{}, DmaMode{}, ic<JF>{}, t);
      substep(ic<2>{}, ic<3>{}, ic<J>{}, DmaMode{}, ic<JF>{}, t);
    }
    wait_vmcnt<VM_WAIT>();
    lds_ring_barrier();
    substep(ic<NSUB - 1>{}, ic<0>{}, ic<JN>{}, DmaLast{}, ic<JF>{}, t);
  };
  // EARLY: substeps 0 and 1 of tile it read sets 2 and 3 (the rest of tile it);
  // then, once this wave's DMA of tile it+1 has landed, a barrier after which
  // no wave reads stage J; substeps 2 and 3 read sets 0 and 1 of tile it+1 and
  // issue the DMA of tile it+2 into stage J, half each.  That DMA has substeps
  // 0 and 1 of the next K tile to land before it is waited for.
  auto iteration4 = [&](auto J_c) __attribute__((always_inline)) {
    constexpr int J = decltype(J_c)::value;
    constexpr int JN = (J + 1) % STAGES;
    const TileRef t = next_tile();
    substep4(ic<0>{}, ic<2>{}, ic<2>{}, ic<J>{}, ic<0>{}, ic<J>{}, t);
    substep4(ic<1>{}, ic<3>{}, ic<3>{}, ic<J>{}, ic<0>{}, ic<J>{}, t);
    wait_vmcnt<0>();
    lds_ring_barrier();
    // The substeps that issue the next tile's DMA run at raised wave priority: the
    // wave that leaves the barrier first keeps the SIMD's issue slot for its MFMAs,
    // reads and DMA instead of alternating with its partner wave instruction by
    // instruction (configuration-3 set +0.8-1 %).
    __builtin_amdgcn_s_setprio(1);
    substep4(ic<2>{}, ic<0>{}, ic<0>{}, ic<JN>{}, ic<1>{}, ic<J>{}, t);
    substep4(ic<3>{}, ic<1>{}, ic<1>{}, ic<JN>{}, ic<2>{}, ic<J>{}, t);
    __builtin_amdgcn_s_setprio(0);
  };
  if constexpr (EARLY) {
    for (int it = it0; it < it1; it += STAGES) static_for<STAGES>(iteration4);
  } else {
    for (int it = it0; it < it1; it += STAGES) static_for<STAGES>(iteration);
  }

  if constexpr (TRR) {
    // The last substep issued transpose reads (asm) for a K tile that does not
    // exist.  Their registers count as dead to the compiler while the reads are
    // still in flight: wait for them, and keep the registers allocated until
    // after the wait so nothing else is placed in them meanwhile.
    __builtin_amdgcn_s_waitcnt(0xC07F);
#pragma unroll
    for (int st = 0; st < (EARLY ? 2 : 1); ++st) {
#pragma unroll
      for (int i = 0; i < TM; ++i) asm volatile("" ::"v"(fa[st][i]));
#pragma unroll
      for (int jj = 0; jj < NB; ++jj) asm volatile("" ::"v"(fb[st][jj]));
    }
  }
  wait_vmcnt<0>();  // DMAs of the all-zero tiles past it1

  // acc[i][j][4q + e] holds C[m][n + e] with
  //   m = m0 + wm*WTM + i*32 + (lane & 31),  n = n0 + wn*WTN + j*32 + 8q + 4*(lane >> 5).
  if constexpr (KG == 2) {
    // Sum the K groups.  The wave of group g keeps row block i = g of its wave
    // tile and sends the other block to its partner (same place in the other
    // group) through LDS, in slots [sender group][wave][j][quad][lane] of 16
    // bytes; the epilogue below then stores only row block kg.
    __syncthreads();  // every wave is past its last fragment read
    static_assert(2 * NWG * TN * 4 * 64 * 16 <= LDS_BYTES, "exchange fits the ring");
    f32x4_t* xb = reinterpret_cast<f32x4_t*>(smem);
    auto slot = [&](int g, int j, int q) __attribute__((always_inline)) {
      return (((g * NWG + wq) * TN + j) * 4 + q) * 64 + lane;
    };
    auto quad = [](const f32x16_t& a, int q) __attribute__((always_inline)) {
      return f32x4_t{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
    };
    auto exchange = [&](auto KEEP_c) __attribute__((always_inline)) {
      constexpr int KEEP = decltype(KEEP_c)::value, SEND = 1 - KEEP;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) xb[slot(KEEP, j, q)] = quad(acc[SEND][j], q);
      __syncthreads();
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4_t r = xb[slot(SEND, j, q)];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[KEEP][j][4 * q + e] += r[e];
        }
    };
    if (kg == 0) exchange(ic<0>{});
    else exchange(ic<1>{});
  }
  auto value = [&](int i, int j, int q, int e) __attribute__((always_inline)) {
    if constexpr (DUAL)
      return silu_f(p.alpha * acc[i][j][4 * q + e]) * (p.alpha * acc[i][j + TN][4 * q + e]);
    else
      return p.alpha * acc[i][j][4 * q + e];
  };
  if constexpr (FAST_EPI) {
    // row scale (a folded RMSNorm): row block i of this lane is row m0 + wm*WTM + 32i +
    // (lane & 31); blocks past M (edge tiles) are not stored and read no scale
    float rsv[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = m0 + wm * WTM + 32 * i + (lane & 31);
      if constexpr (ROWSCALE) rsv[i] = r < p.M ? p.row_scale[r] : 0.0f;
      else rsv[i] = 1.0f;
      (void)r;
    }
    auto scaled = [&](int i, int j, int q, int e) __attribute__((always_inline)) {
      if constexpr (ROWSCALE) return value(i, j, q, e) * rsv[i];
      else return value(i, j, q, e);
    };
    // M and N multiples of 32, epilogue alpha (SiLU gate), beta*C and the output
    // conversion.  Each 32x32 MFMA block goes through a wave-private LDS patch (rows
    // padded by 4 floats) and back out row-major, so a store instruction writes 8
    // rows of 32 contiguous columns (64 or 128 bytes per row) instead of 32 rows of
    // 16 bytes.  A block is wholly inside the matrix or wholly past its edge (an
    // edge tile's extra blocks are skipped).  One barrier first: the patches reuse
    // the ring's LDS (the barrier is in store_tile, after the first beta loads).
    constexpr int PP = 36;  // patch pitch (floats)
    static_assert(NWAVE * 32 * PP * 4 <= LDS_BYTES, "epilogue patches fit the ring");
    float* patch = reinterpret_cast<float*>(smem) + wave * (32 * PP);
    const float beta = p.beta;
    const int r_in = lane & 31, h_in = lane >> 5;
    const int r_out = lane >> 3, c_out = (lane & 7) * 4;  // + 8 rows per step
    // BF: bf16 C; BETA: beta*C is added.  Both uniform, hoisted out of the tile.
    auto store_tile = [&](auto BF_c, auto BETA_c) __attribute__((always_inline)) {
      constexpr bool BF = decltype(BF_c)::value, BETA = decltype(BETA_c)::value;
      // WIDE: patches of 32 x 64 (pitch 68 floats), lane -> row lane / 16, 4 columns
      constexpr int PPW = 68;
      constexpr bool WIDE = BF && !BETA && TN % 2 == 0 && KG == 1 && NWAVE * 32 * PPW * 4 <= LDS_BYTES;
      float* patchw = reinterpret_cast<float*>(smem) + wave * (32 * PPW);
      const int rw_out = lane >> 4, cw_out = (lane & 15) * 4;
      using OldT = std::conditional_t<BF, u32x2_t, f32x4_t>;
      auto col_of = [&](int j) __attribute__((always_inline)) { return n0 + wn * WTN + j * 32 + c_out; };
      auto row_of = [&](int i) __attribute__((always_inline)) {
        return (int64_t)(m0 + wm * WTM + i * 32 + r_out);
      };
      auto inside = [&](int j) __attribute__((always_inline)) {
        return uniform(n0 + wn * WTN + j * 32) < p.N;
      };
      auto valid = [&](int i) __attribute__((always_inline)) {  // row block i stored by this wave
        return (KG == 1 || i == kg) && uniform(m0 + wm * WTM + i * 32) < p.M;
      };
      // beta: the old C of row block i + 1 is loaded while row block i is stored (row
      // block 0's before the barrier), so the load latency overlaps other work
      OldT old[2][TN][4];
      auto load_old = [&](int i, OldT (&dst)[TN][4]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (!inside(j)) continue;
#pragma unroll
          for (int st = 0; st < 4; ++st) {
            const int64_t ci = (row_of(i) + 8 * st) * p.ldc + col_of(j);
            // non-temporal: the old C is read once (configuration-3 set with its fp32 beta = 1
            // weight gradients 1144-1146 -> 1163-1164 TFLOP/s, one box)
            if constexpr (BF) dst[j][st] = __builtin_nontemporal_load((const u32x2_t*)((const uint16_t*)Cz + ci));
            else dst[j][st] = __builtin_nontemporal_load((const f32x4_t*)((const float*)Cz + ci));
          }
        }
      };
      if constexpr (BETA) {
        if (valid(0)) load_old(0, old[0]);
      }
      __syncthreads();  // the patches reuse the ring's LDS
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        if constexpr (BETA) {
          if (i + 1 < TM && valid(i + 1)) load_old(i + 1, old[(i + 1) & 1]);
        }
        if (!valid(i)) continue;
        if constexpr (WIDE) {
          // bf16 without beta: two 32x32 blocks per patch, read back as 4 rows of 64
          // columns, so every store instruction writes whole 128-byte rows (configuration-3
          // set 1171-1173 -> 1181-1183 TFLOP/s, LM head 1203 -> 1222, one box)
#pragma unroll
          for (int jp = 0; jp < TN; jp += 2) {
            if (!inside(jp)) continue;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                f32x4_t v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = scaled(i, jp + h, q, e);
                *reinterpret_cast<f32x4_t*>(patchw + r_in * PPW + 32 * h + 8 * q + 4 * h_in) = v;
              }
            const int colw = n0 + wn * WTN + jp * 32 + cw_out;
            const bool ok = cw_out < 32 || inside(jp + 1);  // the second block may lie past N
            const int64_t roww = m0 + wm * WTM + i * 32 + rw_out;
#pragma unroll
            for (int st = 0; st < 8; ++st) {
              const f32x4_t v = *reinterpret_cast<const f32x4_t*>(patchw + (rw_out + 4 * st) * PPW + cw_out);
              const int64_t ci = (roww + 4 * st) * p.ldc + colw;
              if (ok)
                __builtin_nontemporal_store(u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])},
                                            (u32x2_t*)((uint16_t*)Cz + ci));
            }
            __builtin_amdgcn_sched_barrier(0);
          }
          continue;
        }
        const int64_t row0 = row_of(i);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (!inside(j)) continue;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            f32x4_t v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = scaled(i, j, q, e);
            *reinterpret_cast<f32x4_t*>(patch + r_in * PP + 8 * q + 4 * h_in) = v;
          }
          const int col = col_of(j);
#pragma unroll
          for (int st = 0; st < 4; ++st) {
            f32x4_t v = *reinterpret_cast<const f32x4_t*>(patch + (r_out + 8 * st) * PP + c_out);
            const int64_t ci = (row0 + 8 * st) * p.ldc + col;
            if constexpr (BF) {
              if constexpr (BETA) {
                const u32x2_t o = old[i & 1][j][st];
                v[0] += beta * bf16_bits_to_f32(o[0] & 0xffffu);
                v[1] += beta * bf16_bits_to_f32(o[0] >> 16);
                v[2] += beta * bf16_bits_to_f32(o[1] & 0xffffu);
                v[3] += beta * bf16_bits_to_f32(o[1] >> 16);
              }
              // non-temporal: C streams out instead of filling the XCD's L2 with dirty lines
              // (configuration-3 set 1133-1134 -> 1141-1144 TFLOP/s, down forward +4 %, one box)
              __builtin_nontemporal_store(u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])},
                                          (u32x2_t*)((uint16_t*)Cz + ci));
            } else {
              if constexpr (BETA) {
                const f32x4_t o = old[i & 1][j][st];
                v[0] += beta * o[0]; v[1] += beta * o[1];
                v[2] += beta * o[2]; v[3] += beta * o[3];
              }
              __builtin_nontemporal_store(v, (f32x4_t*)((float*)Cz + ci));
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    if (p.c_bf16) {
      if (beta != 0.0f) store_tile(std::true_type{}, std::true_type{});
      else store_tile(std::true_type{}, std::false_type{});
    } else {
      if (beta != 0.0f) store_tile(std::false_type{}, std::true_type{});
      else store_tile(std::false_type{}, std::false_type{});
    }
  } else {

  // General epilogue (bias, residual, causal mask, edge tiles, split-K
  // partials): each 32-row block of the wave tile is staged through LDS (rows
  // padded by 4 floats) and walked row-major by a rolled loop around one
  // epilogue4.  The staging area is private to the wave, so only the first use
  // of the ring's LDS needs every wave past its last fragment read.
  __syncthreads();
  constexpr int PITCH = WTN + 4;
  static_assert(NWAVE * 32 * PITCH * 4 <= LDS_BYTES, "epilogue staging fits the ring");
  float* stg = reinterpret_cast<float*>(smem) + wave * (32 * PITCH);
  float* W = (p.splits > 1) ? p.ws + ((int64_t)tc.z * p.splits + tc.split) * (int64_t)p.M * p.N
                            : nullptr;
  const int lrow = lane & 31, lhalf = lane >> 5;
  constexpr int C4 = WTN / 4;  // float4 groups per staged row
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    if (KG == 2 && i != kg) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4_t v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = DUAL ? value(i, j, q, e) : acc[i][j][4 * q + e];
        *reinterpret_cast<f32x4_t*>(stg + lrow * PITCH + j * 32 + 8 * q + 4 * lhalf) = v;
      }
    __builtin_amdgcn_sched_barrier(0);
    const int mrow0 = m0 + wm * WTM + i * 32;
    const int ncol0 = n0 + wn * WTN;
#pragma unroll 1
    for (int idx = lane; idx < 32 * C4; idx += 64) {
      const int r = idx / C4, c4 = idx % C4;
      const f32x4_t sv = *reinterpret_cast<const f32x4_t*>(stg + r * PITCH + c4 * 4);
      const int m = mrow0 + r, n = ncol0 + c4 * 4;
      if (W) {
        // split-K partials: alpha is applied by the reduction
        if (m < p.M) {
          if ((p.N & 3) == 0 && n + 3 < p.N) {
            *reinterpret_cast<f32x4_t*>(W + (int64_t)m * p.N + n) = sv;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < p.N) W[(int64_t)m * p.N + n + e] = sv[e];
          }
        }
      } else {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = DUAL ? sv[e] : p.alpha * sv[e];
        epilogue4(p, Cz, Rz, m, n, v);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  }
}

}  // namespace mig
