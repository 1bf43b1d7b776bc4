// mi_gemm_device.hpp -- device code of the gfx950 GEMM core.
//
// One kernel template covers every matmul of the reference engine's decoder
// block (Tensor::matmul, Tensor.cpp:174-228, and the metal_bridge GEMM entry
// points, MetalBridge.hpp:39-46,119-125):
//   * bf16 inputs -> v_mfma_f32_32x32x16_bf16, fp32 inputs -> v_mfma_f32_32x32x2f32,
//     fp32 accumulation in both cases;
//   * any transpose combination: an operand whose K index is contiguous in memory
//     ("K-contiguous") is copied chunk-for-chunk into LDS; an operand whose M/N
//     index is contiguous is loaded as 16-byte rows of a small (k x row) block and
//     transposed in registers before the LDS write, so LDS always holds
//     [row][K-tile] tiles and the MFMA fragments are single ds_read_b128s;
//   * LDS rows are 128 bytes (64 bf16 / 32 fp32) in 16-byte chunks whose position
//     is XOR-swizzled by the row, so the fragment reads (16 consecutive rows per
//     LDS cycle, one chunk column) and the tile writes are bank-conflict free;
//   * two LDS buffers: global loads for tile k+1 are issued into registers before
//     the MFMAs of tile k, stored to the other buffer after, one barrier per tile;
//   * fused epilogue (alpha, bias, beta*C, residual, bf16/fp32 output, causal
//     mask), dual-B SiLU-gate (gemm_ffn.metal:160-181) and SiLU-gate A prologue
//     (fused_swiglu_gemm.metal:48-77);
//   * strided batches with a GQA head->kv-head map and K segments (the KV-group
//     reduction of Attention.cpp:332,344-345) and causal tile skipping;
//   * split-K over a caller workspace, reduced deterministically by a second kernel.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace mig {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

enum { MODE_PLAIN = 0, MODE_DUAL = 1, MODE_PROLOGUE = 2 };
enum { CAUSAL_NONE = 0, CAUSAL_OUT_LOWER = 1, CAUSAL_A_LOWER = 2, CAUSAL_A_UPPER = 3 };

struct Params {
  const void* A;
  const void* A2;
  const void* B;
  const void* B2;
  void* C;
  const void* bias;
  const void* R;
  float* ws;
  int64_t lda, ldb, ldc, ldr;
  int64_t segA, segB;
  int64_t aO, aI, bO, bI, cO, cI, rO, rI;
  int M, N, K, nseg;
  int heads, gA, gB, gC;
  int tiles_m, tiles_n, splits, batch;
  int causal;
  float mask_value;
  float alpha, beta;
  int c_bf16, bias_bf16, r_bf16;
  int vecA, vecB;  // 16-byte global loads legal for A (and A2) / B (and B2)
  int cvec;        // 4-wide C / R / bias accesses legal
  uint32_t extA, extB;  // byte extent of one batch/segment matrix of A (A2) / B (B2)
  const float* row_scale;  // optional [M] fp32 factor on row m of alpha * acc (a folded RMSNorm)
  int krot;             // direct-to-LDS kernels: start each XCD's tiles at its own K offset
  int group_m;          // tile rows per column sweep of the tile order (map_tile)
};

// ---------------------------------------------------------------------------
// scalar helpers

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two floats to packed bf16 (lo in bits 15:0): one v_cvt_pk_bf16_f32, which
// rounds to nearest even and keeps NaN a NaN.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) { return pack_bf16x2(f, 0.0f) & 0xffffu; }

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }

// Chunk position of chunk c (0..7) in LDS row r.  For any 16 consecutive rows
// read at one chunk column, (r & 1, position) is distinct, and for any 8
// consecutive rows the position is distinct: conflict-free for both a 32-bank
// and a 64-bank 4-byte LDS.
#ifndef MI_SWZ
#define MI_SWZ 0
#endif
__device__ __forceinline__ int swz(int r, int c) {
#if MI_SWZ == 0
  return c ^ ((r ^ (r >> 3)) & 7);
#elif MI_SWZ == 1
  return c ^ (r & 7);
#elif MI_SWZ == 2
  return c ^ ((r >> 1) & 7);
#else
  return c;
#endif
}

template <typename T>
struct ElemTraits;
template <>
struct ElemTraits<float> {
  static constexpr int CH = 4;  // elements per 16-byte chunk
  __device__ static uint32_t bits(const void* p, int64_t i) { return ((const uint32_t*)p)[i]; }
};
template <>
struct ElemTraits<__bf16> {
  static constexpr int CH = 8;
  __device__ static uint32_t bits(const void* p, int64_t i) { return ((const uint16_t*)p)[i]; }
};

// Pack CH scalar bit patterns into a 16-byte chunk.
template <typename T>
__device__ __forceinline__ u32x4_t pack_chunk(const uint32_t* e) {
  u32x4_t v;
  if constexpr (sizeof(T) == 4) {
    v[0] = e[0]; v[1] = e[1]; v[2] = e[2]; v[3] = e[3];
  } else {
    v[0] = e[0] | (e[1] << 16); v[1] = e[2] | (e[3] << 16);
    v[2] = e[4] | (e[5] << 16); v[3] = e[6] | (e[7] << 16);
  }
  return v;
}

// Load the 16-byte chunk of CH consecutive elements starting at element index
// `i` of `p`, `n_ok` of which are in bounds (0..CH).  vec: the chunk is
// 16-byte aligned and the fast path may be used.
template <typename T>
__device__ __forceinline__ u32x4_t load_chunk(const void* p, int64_t i, int n_ok, bool vec) {
  constexpr int CH = ElemTraits<T>::CH;
  if (n_ok >= CH && vec) return *(const u32x4_t*)((const T*)p + i);
  uint32_t e[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) e[j] = (j < n_ok) ? ElemTraits<T>::bits(p, i + j) : 0u;
  return pack_chunk<T>(e);
}

// SiLU(g)*u on a chunk pair, re-encoded in T.
template <typename T>
__device__ __forceinline__ u32x4_t swiglu_chunk(u32x4_t g, u32x4_t u) {
  u32x4_t o;
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = __float_as_uint(silu_f(__uint_as_float(g[j])) * __uint_as_float(u[j]));
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float g0 = bf16_bits_to_f32(g[j] & 0xffffu), g1 = bf16_bits_to_f32(g[j] >> 16);
      const float u0 = bf16_bits_to_f32(u[j] & 0xffffu), u1 = bf16_bits_to_f32(u[j] >> 16);
      o[j] = pack_bf16x2(silu_f(g0) * u0, silu_f(g1) * u1);
    }
  }
  return o;
}

// ---------------------------------------------------------------------------
// Tile loader: R rows x KT (= 8 chunks) of one operand, global -> registers -> LDS.
//   KC = true : element (r, k) at r*ld + k   (K-contiguous)
//   KC = false: element (r, k) at k*ld + r   (row-contiguous; transposed in registers)
// PRO (prologue): the operand is SiLU(X) * X2, computed at LDS-store time.
// FAST: buffer loads through a resource descriptor whose num_records is the
//   operand's byte extent.  Offsets past the extent return zero in hardware, so
//   rows past the matrix edge (K-contiguous) and K past the edge (row-contiguous)
//   need no code; the remaining edge (K tail of a K-contiguous row, row tail of a
//   row-contiguous k line) is sent to an offset past the extent.  Every chunk is
//   one branch-free buffer_load_dwordx4.  Requires every chunk fully inside or
//   fully outside the matrix, 16-byte alignment and 31-bit byte offsets (checked
//   on the host).
// !FAST: element-granular bounds for any shape, leading dimension or alignment.

constexpr uint32_t kBufOOB = 0x80000000u;          // offset past any extent < 2^31
constexpr int kBufFlags = 0x00020000;               // raw-buffer dword3 for gfx9-family

// Values that are uniform across the workgroup but which the compiler may have
// computed in vector registers (integer division lowers through VALU).  Moving
// them to scalar registers keeps buffer descriptors scalar: a descriptor the
// compiler believes divergent is wrapped in a per-load waterfall loop.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

template <typename P>
__device__ __forceinline__ P* uniform(P* ptr) {
  const uint64_t v = (uint64_t)ptr;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (P*)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t ext) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(uniform(base)), (short)0,
                                           (int)uniform((int)ext), kBufFlags);
}

__device__ __forceinline__ u32x4_t buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, 0);
}

template <typename T, int R, bool KC, bool PRO, bool FAST>
struct TileLoader {
  static constexpr int CH = ElemTraits<T>::CH;
  static constexpr int ESZ = (int)sizeof(T);
  static constexpr int NT = 256;
  // K-contiguous: R*8 chunks over 256 threads.
  static constexpr int NCK = (R * 8 + NT - 1) / NT;
  // Row-contiguous: 8*(R/CH) blocks of CH x CH, each CH chunks.
  static constexpr int NBLK_TOT = 8 * (R / CH);
  static constexpr int NBLK = (NBLK_TOT + NT - 1) / NT;
  // Work is issued in units so the main loop can spread it between MFMAs:
  // a load unit is one 16-byte chunk load; a store unit is one 16-byte LDS write
  // (for a row-contiguous operand: one row of a transposed block).
  static constexpr int NUNIT = KC ? NCK : NBLK * CH;
  u32x4_t st[NUNIT];
  u32x4_t st2[PRO ? NUNIT : 1];
  // fast path: per-thread byte offsets fixed for the tile
  uint32_t off0;                  // KC: chunk 0 of this thread at k = 0
  uint32_t boff[KC ? 1 : NBLK];   // !KC: block i at k = 0 (>= 2^31 when its rows are outside)
  int ldb;                        // leading dimension in bytes
  int koff;                       // KC: this thread's chunk column * CH
  int rows_, row0_;
  int64_t ld_;
  // per K tile
  __amdgpu_buffer_rsrc_t rs, rs2;
  const void* base_;
  const void* base2_;
  uint32_t kv0, kmask;
  int k0_, kseg_;
  bool vec_;

  __device__ __forceinline__ void init(int64_t ld, int rows, int row0) {
    const int tid = threadIdx.x;
    rows_ = rows;
    row0_ = row0;
    ld_ = ld;
    if constexpr (FAST) {
      ldb = (int)ld * ESZ;
      if constexpr (KC) {
        koff = (tid & 7) * CH;
        off0 = (uint32_t)((row0 + (tid >> 3)) * ldb + koff * ESZ);
      } else {
#pragma unroll
        for (int i = 0; i < NBLK; ++i) {
          const int b = tid + NT * i;
          const int rb = b % (R / CH), kb = b / (R / CH);
          const int grow = row0 + rb * CH;
          boff[i] = (b < NBLK_TOT && grow < rows) ? (uint32_t)(grow * ESZ + kb * CH * ldb) : kBufOOB;
        }
      }
    }
  }

  // Select the K tile: base/base2 are the operand pointers of the current batch
  // and K segment, ext their byte extent, k0 the tile's first K, kseg the K extent.
  // live = false turns every load of the tile into an out-of-range no-op.
  __device__ __forceinline__ void set_tile(const void* base, const void* base2, uint32_t ext, int k0,
                                           int kseg, bool vec, bool live) {
    k0_ = k0;
    kseg_ = live ? kseg : 0;
    if constexpr (FAST) {
      (void)vec;
      rs = make_rsrc(base, ext);
      if constexpr (PRO) rs2 = make_rsrc(base2, ext);
      // offsets stay below 2^31, so OR-ing the top bit moves a chunk out of range
      if constexpr (KC) {
        kmask = (live && koff + k0 < kseg) ? 0u : kBufOOB;
        kv0 = off0 + (uint32_t)(k0 * ESZ);
      } else {
        kmask = live ? 0u : kBufOOB;
      }
    } else {
      (void)ext;
      base_ = base;
      base2_ = base2;
      vec_ = vec;
    }
  }

  __device__ __forceinline__ void load_unit(int u) {
    const int tid = threadIdx.x;
    if constexpr (FAST) {
      if constexpr (KC) {
        const uint32_t vo = (kv0 + (uint32_t)(u * 32 * ldb)) | kmask;
        st[u] = buf_load16(rs, vo);
        if constexpr (PRO) st2[u] = buf_load16(rs2, vo);
      } else {
        const int i = u / CH, kk = u % CH;
        // boff[i] >= 2^31 for rows outside; adding < 2^31 keeps it outside
        const uint32_t vo = (boff[i] + (uint32_t)((k0_ + kk) * ldb)) | kmask;
        st[u] = buf_load16(rs, vo);
        if constexpr (PRO) st2[u] = buf_load16(rs2, vo);
      }
    } else {
      if constexpr (KC) {
        const int idx = tid + NT * u;
        const int r = idx >> 3, c = idx & 7;
        const int grow = row0_ + r, gk = k0_ + c * CH;
        int n_ok = (grow < rows_ && idx < R * 8) ? kseg_ - gk : 0;
        n_ok = n_ok < 0 ? 0 : (n_ok > CH ? CH : n_ok);
        const int64_t off = (int64_t)grow * ld_ + gk;
        st[u] = load_chunk<T>(base_, off, n_ok, vec_);
        if constexpr (PRO) st2[u] = load_chunk<T>(base2_, off, n_ok, vec_);
      } else {
        const int i = u / CH, kk = u % CH;
        const int b = tid + NT * i;
        const int rb = b % (R / CH), kb = b / (R / CH);
        const int grow = row0_ + rb * CH;
        int n_ok = (b < NBLK_TOT) ? rows_ - grow : 0;
        n_ok = n_ok < 0 ? 0 : (n_ok > CH ? CH : n_ok);
        const int gk = k0_ + kb * CH + kk;
        const int nk = (gk < kseg_) ? n_ok : 0;
        const int64_t off = (int64_t)gk * ld_ + grow;
        st[u] = load_chunk<T>(base_, off, nk, vec_);
        if constexpr (PRO) st2[u] = load_chunk<T>(base2_, off, nk, vec_);
      }
    }
  }

  // lds: this operand's region, R rows of 8 chunks.
  __device__ __forceinline__ void store_unit(int u, u32x4_t* lds) {
    const int tid = threadIdx.x;
    if constexpr (KC) {
      const int idx = tid + NT * u;
      if (NCK * NT == R * 8 || idx < R * 8) {
        const int r = idx >> 3, c = idx & 7;
        u32x4_t v = st[u];
        if constexpr (PRO) v = swiglu_chunk<T>(st[u], st2[u]);
        lds[r * 8 + swz(r, c)] = v;
      }
    } else {
      const int i = u / CH, j = u % CH;
      const int b = tid + NT * i;
      if (NBLK * NT == NBLK_TOT || b < NBLK_TOT) {
        const int rb = b % (R / CH), kb = b / (R / CH);
        // row j of the transposed block: element j of each of the CH k-chunks
        u32x4_t o;
        if constexpr (sizeof(T) == 4) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) o[kk] = st[i * CH + kk][j];
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t a = st[i * CH + 2 * q][j >> 1], bb = st[i * CH + 2 * q + 1][j >> 1];
            o[q] = (j & 1) ? ((a >> 16) | (bb & 0xffff0000u)) : ((a & 0xffffu) | (bb << 16));
          }
        }
        const int r = rb * CH + j;
        lds[r * 8 + swz(r, kb)] = o;
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Epilogue for 4 consecutive columns n..n+3 of row m.  v holds the finished
// alpha-scaled (or SiLU-gated) accumulator values.

__device__ __forceinline__ float ld_any(const void* p, int64_t i, int is_bf16) {
  return is_bf16 ? bf16_bits_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

__device__ __forceinline__ void epilogue4(const Params& p, void* Cz, const void* Rz, int m, int n,
                                          float v[4]) {
  if (m >= p.M || n >= p.N) return;
  if (p.row_scale) {
    const float s = p.row_scale[m];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] *= s;
  }
  const bool full = (n + 3 < p.N) && p.cvec;
  const int64_t ci = (int64_t)m * p.ldc + n;
  if (p.bias) {
    if (full) {
      if (p.bias_bf16) {
        const u32x2_t b = *(const u32x2_t*)((const uint16_t*)p.bias + n);
        v[0] += bf16_bits_to_f32(b[0] & 0xffffu); v[1] += bf16_bits_to_f32(b[0] >> 16);
        v[2] += bf16_bits_to_f32(b[1] & 0xffffu); v[3] += bf16_bits_to_f32(b[1] >> 16);
      } else {
        const f32x4_t b = *(const f32x4_t*)((const float*)p.bias + n);
        v[0] += b[0]; v[1] += b[1]; v[2] += b[2]; v[3] += b[3];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < p.N) v[e] += ld_any(p.bias, n + e, p.bias_bf16);
    }
  }
  if (p.beta != 0.0f) {
    if (full) {
      if (p.c_bf16) {
        const u32x2_t c = *(const u32x2_t*)((const uint16_t*)Cz + ci);
        v[0] += p.beta * bf16_bits_to_f32(c[0] & 0xffffu);
        v[1] += p.beta * bf16_bits_to_f32(c[0] >> 16);
        v[2] += p.beta * bf16_bits_to_f32(c[1] & 0xffffu);
        v[3] += p.beta * bf16_bits_to_f32(c[1] >> 16);
      } else {
        const f32x4_t c = *(const f32x4_t*)((const float*)Cz + ci);
        v[0] += p.beta * c[0]; v[1] += p.beta * c[1];
        v[2] += p.beta * c[2]; v[3] += p.beta * c[3];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < p.N) v[e] += p.beta * ld_any(Cz, ci + e, p.c_bf16);
    }
  }
  if (Rz) {
    const int64_t ri = (int64_t)m * p.ldr + n;
    if (full) {
      if (p.r_bf16) {
        const u32x2_t r = *(const u32x2_t*)((const uint16_t*)Rz + ri);
        v[0] += bf16_bits_to_f32(r[0] & 0xffffu); v[1] += bf16_bits_to_f32(r[0] >> 16);
        v[2] += bf16_bits_to_f32(r[1] & 0xffffu); v[3] += bf16_bits_to_f32(r[1] >> 16);
      } else {
        const f32x4_t r = *(const f32x4_t*)((const float*)Rz + ri);
        v[0] += r[0]; v[1] += r[1]; v[2] += r[2]; v[3] += r[3];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < p.N) v[e] += ld_any(Rz, ri + e, p.r_bf16);
    }
  }
  if (p.causal == CAUSAL_OUT_LOWER) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n + e > m) v[e] = p.mask_value;
  }
  if (full) {
    if (p.c_bf16) {
      u32x2_t o;
      o[0] = pack_bf16x2(v[0], v[1]);
      o[1] = pack_bf16x2(v[2], v[3]);
      *(u32x2_t*)((uint16_t*)Cz + ci) = o;
    } else {
      f32x4_t o = {v[0], v[1], v[2], v[3]};
      *(f32x4_t*)((float*)Cz + ci) = o;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (n + e < p.N) {
        if (p.c_bf16)
          ((uint16_t*)Cz)[ci + e] = (uint16_t)f32_to_bf16_rne(v[e]);
        else
          ((float*)Cz)[ci + e] = v[e];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Work decomposition shared by the GEMM and the split-K reduction.

struct TileCoord {
  int z, split, tm, tn;
};

// Hardware hands workgroup b to XCD (b mod 8).  Renumber so each XCD receives a
// contiguous range of logical tiles, then order tiles in groups of group_m tile
// rows so that the workgroups resident on one XCD share A and B panels in its L2.
#ifndef MI_GROUP_M
#define MI_GROUP_M 8
#endif
#ifndef MI_XCD_REMAP
#define MI_XCD_REMAP 1
#endif
#ifndef MI_SCHED
#define MI_SCHED 0
#endif

__device__ __forceinline__ TileCoord map_tile(int bid, int nblocks, int tiles_m, int tiles_n,
                                              int splits, int causal, int group_m) {
  constexpr int NXCD = 8;
  const int GROUP_M = group_m;
  if (causal == CAUSAL_A_LOWER || causal == CAUSAL_A_UPPER) {
    // Causal-skipping products: a tile's K range grows with its row block (A_LOWER)
    // or shrinks with it (A_UPPER).  Workgroups are dispatched in block order, so
    // handing out the longest row blocks of every problem first lets the short ones
    // fill the tail (longest processing time first) instead of a long tile starting
    // last.  Consecutive blocks cycle over the XCDs, each of which gets the same mix.
    const int per = nblocks / tiles_m;  // problems x splits x column blocks per row block
    const int r = bid / per, rest = bid - r * per;
    TileCoord tc;
    tc.tm = causal == CAUSAL_A_LOWER ? tiles_m - 1 - r : r;
    tc.tn = rest % tiles_n;
    const int zs = rest / tiles_n;
    tc.z = zs / splits;
    tc.split = zs - tc.z * splits;
    return tc;
  }
#if MI_XCD_REMAP
  const int q = nblocks / NXCD, rem = nblocks % NXCD;
  const int x = bid % NXCD, j = bid / NXCD;
  const int lid = x * q + (x < rem ? x : rem) + j;
#else
  const int lid = bid;
#endif
  const int tiles = tiles_m * tiles_n;
  TileCoord tc;
  const int zs = lid / tiles;
  int t = lid - zs * tiles;
  tc.z = zs / splits;
  tc.split = zs - tc.z * splits;
  const int group = GROUP_M * tiles_n;
  const int g = t / group;
  const int first_m = g * GROUP_M;
  const int gm = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
  t -= g * group;
  tc.tm = first_m + t % gm;
  tc.tn = t / gm;
  return tc;
}

// ---------------------------------------------------------------------------
// The GEMM kernel.
//   AK: A is K-contiguous (transA == 0).   BK: B is K-contiguous (transB == 1).
//   Tile BM x BN (output), KT = 8 chunks of K per LDS stage, 4 waves in a
//   WGM x WGN grid, each wave computing a (BM/WGM) x (BN/WGN) block from 32x32
//   MFMA tiles.  MODE_DUAL keeps a second accumulator set for B2 (LDS B region
//   holds 2*BN rows: B then B2).
//
// Main loop (two LDS buffers, one barrier per K tile, fragments double-buffered
// in registers):
//   issue global loads of tile k+1
//   substeps 0..2:  read fragments of substep s+1 | MFMAs of substep s
//   store tile k+1 to the other LDS buffer;  barrier
//   read fragments of substep 0 of tile k+1 | MFMAs of substep 3 of tile k
// so the LDS latency after the barrier hides under the last substep's MFMAs.

template <typename T, int BM, int BN, int WGM, int WGN, bool AK, bool BK, int MODE, bool FAST>
__global__ void __launch_bounds__(256)
    __attribute__((amdgpu_waves_per_eu(BM * BN >= 256 * 128 ? 1 : 2)))
    gemm_kernel(Params p) {
  constexpr int CH = ElemTraits<T>::CH;
  constexpr int KT = 8 * CH;
  constexpr int BROWS = (MODE == MODE_DUAL) ? 2 * BN : BN;
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int NB = (MODE == MODE_DUAL) ? 2 * TN : TN;
  constexpr bool PRO = (MODE == MODE_PROLOGUE);
  static_assert(WGM * WGN == 4, "4 waves per workgroup");
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold one 32x32 MFMA tile");

  __shared__ u32x4_t smem[2][(BM + BROWS) * 8];

  const int nblocks = gridDim.x;
  const TileCoord tc = map_tile(blockIdx.x, nblocks, p.tiles_m, p.tiles_n, p.splits, p.causal, p.group_m);
  const int m0 = uniform(tc.tm * BM), n0 = uniform(tc.tn * BN);
  const int zo = uniform(tc.z / p.heads), zi = uniform(tc.z - (tc.z / p.heads) * p.heads);
  const int ziA = uniform(zi / p.gA), ziB = uniform(zi / p.gB), ziC = uniform(zi / p.gC);
  const T* Ab = uniform((const T*)p.A + (int64_t)zo * p.aO + (int64_t)ziA * p.aI);
  const T* A2b = PRO ? uniform((const T*)p.A2 + (int64_t)zo * p.aO + (int64_t)ziA * p.aI) : nullptr;
  const T* Bb = uniform((const T*)p.B + (int64_t)zo * p.bO + (int64_t)ziB * p.bI);
  const T* B2b = (MODE == MODE_DUAL) ? uniform((const T*)p.B2 + (int64_t)zo * p.bO + (int64_t)ziB * p.bI)
                                      : nullptr;
  const int64_t coff = (int64_t)zo * p.cO + (int64_t)ziC * p.cI;
  const int esz_c = p.c_bf16 ? 2 : 4;
  void* Cz = (char*)p.C + coff * esz_c;
  const void* Rz = p.R ? (const char*)p.R + ((int64_t)zo * p.rO + (int64_t)zi * p.rI) * (p.r_bf16 ? 2 : 4)
                       : nullptr;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WGN, wn = wave % WGN;

  // Fully masked causal tile: only the mask value is written.
  if (p.causal == CAUSAL_OUT_LOWER && n0 > m0 + BM - 1) {
    if (p.splits > 1) return;  // the reduction kernel writes the mask
    for (int idx = threadIdx.x; idx < BM * BN; idx += 256) {
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

  // K iteration space: per segment, K tiles [klo, khi); causal skipping.
  const int kt_seg = (p.K + KT - 1) / KT;
  int klo = 0, khi = kt_seg;
  if (p.causal == CAUSAL_A_LOWER) {
    const int lim = (m0 + BM + KT - 1) / KT;
    khi = khi < lim ? khi : lim;
  } else if (p.causal == CAUSAL_A_UPPER) {
    klo = m0 / KT;
  }
  const int per_seg = khi > klo ? khi - klo : 0;
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

  TileLoader<T, BM, AK, PRO, FAST> la;
  TileLoader<T, BN, BK, false, FAST> lb;
  TileLoader<T, (MODE == MODE_DUAL) ? BN : 32, BK, false, FAST> lb2;
  la.init(p.lda, p.M, m0);
  lb.init(p.ldb, p.N, n0);
  if constexpr (MODE == MODE_DUAL) lb2.init(p.ldb, p.N, n0);

  // Point the loaders at K tile `it` (clamped into range; a tile past it1 is
  // loaded as out-of-range no-ops so the main loop needs no branches).
  auto set_tiles = [&](int it) {
    const bool live = it < it1;
    const int itc = live ? it : it1 - 1;
    const int seg = itc / per_seg;
    const int k0 = (klo + (itc - seg * per_seg)) * KT;
    la.set_tile(Ab + (int64_t)seg * p.segA, PRO ? (const void*)(A2b + (int64_t)seg * p.segA) : nullptr,
                p.extA, k0, p.K, p.vecA, live);
    lb.set_tile(Bb + (int64_t)seg * p.segB, nullptr, p.extB, k0, p.K, p.vecB, live);
    if constexpr (MODE == MODE_DUAL)
      lb2.set_tile(B2b + (int64_t)seg * p.segB, nullptr, p.extB, k0, p.K, p.vecB, live);
  };
  constexpr int NLA = TileLoader<T, BM, AK, PRO, FAST>::NUNIT;
  constexpr int NLB = TileLoader<T, BN, BK, false, FAST>::NUNIT;
  constexpr int NLB2 = (MODE == MODE_DUAL) ? NLB : 0;
  constexpr int NUNITS = NLA + NLB + NLB2;
  auto load_op = [&](int o) {
    if (o < NLA) la.load_unit(o);
    else if (o < NLA + NLB) lb.load_unit(o - NLA);
    else lb2.load_unit(o - NLA - NLB);
  };
  auto store_op = [&](int o, int buf) {
    if (o < NLA) la.store_unit(o, &smem[buf][0]);
    else if (o < NLA + NLB) lb.store_unit(o - NLA, &smem[buf][BM * 8]);
    else lb2.store_unit(o - NLA - NLB, &smem[buf][(BM + BN) * 8]);
  };

  const int lrow = lane & 31, lhalf = lane >> 5;
  // Fragment register sets: fa/fb[set][tile]; substep s uses set s & 1.
  u32x4_t fa[2][TM], fb[2][NB];
  constexpr int NREAD = TM + NB;
  auto read_op = [&](int o, int buf, int s, int set) {
    const int c = 2 * s + lhalf;
    if (o < TM) {
      const int r = wm * WTM + o * 32 + lrow;
      fa[set][o] = smem[buf][r * 8 + swz(r, c)];
    } else {
      const int j = o - TM;
      const int half = (MODE == MODE_DUAL) ? (j / TN) : 0;
      const int jj = (MODE == MODE_DUAL) ? (j % TN) : j;
      const int r = BM + half * BN + wn * WTN + jj * 32 + lrow;
      fb[set][j] = smem[buf][r * 8 + swz(r, c)];
    }
  };
  auto mfma_op = [&](int set, int i, int j) {
    if constexpr (sizeof(T) == 2) {
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          __builtin_bit_cast(bf16x8_t, fb[set][j]), __builtin_bit_cast(bf16x8_t, fa[set][i]),
          acc[i][j], 0, 0, 0);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
            __uint_as_float(fb[set][j][e]), __uint_as_float(fa[set][i][e]), acc[i][j], 0, 0, 0);
    }
  };

  // One substep: TM*NB MFMA slots.  Each slot holds one MFMA (one 32x32 output
  // tile, 16 K) and an even share of the side work of this substep: the
  // fragment reads of the next substep, and in substep 2 the LDS stores of the
  // next K tile, in substep 3 the global loads of the K tile after it.  The
  // scheduling fence after every slot keeps this order, so the wave never
  // waits on an LDS read or a global load it issued in the same slot.
  constexpr int NS = TM * NB;
  auto substep = [&](auto S_c, int rbuf, int sbuf) {
    constexpr int S = decltype(S_c)::value;
    constexpr int set = S & 1, rset = (S + 1) & 1, rs_sub = (S + 1) & 3;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      mfma_op(set, q / NB, q % NB);
#pragma unroll
      for (int o = (q * NREAD + NS - 1) / NS; o < ((q + 1) * NREAD + NS - 1) / NS; ++o)
        read_op(o, rbuf, rs_sub, rset);
      if constexpr (S == 2) {
#pragma unroll
        for (int o = (q * NUNITS + NS - 1) / NS; o < ((q + 1) * NUNITS + NS - 1) / NS; ++o)
          store_op(o, sbuf);
      }
      if constexpr (S == 3) {
#pragma unroll
        for (int o = (q * NUNITS + NS - 1) / NS; o < ((q + 1) * NUNITS + NS - 1) / NS; ++o)
          load_op(o);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Prologue: tile it0 into LDS buffer 0, tile it0+1 into the staging registers,
  // fragments of substep 0.
  if (it0 < it1) {
    set_tiles(it0);
#pragma unroll
    for (int o = 0; o < NUNITS; ++o) load_op(o);
#pragma unroll
    for (int o = 0; o < NUNITS; ++o) store_op(o, 0);
    set_tiles(it0 + 1);
#pragma unroll
    for (int o = 0; o < NUNITS; ++o) load_op(o);
  }
  __syncthreads();
  if (it0 < it1) {
#pragma unroll
    for (int o = 0; o < NREAD; ++o) read_op(o, 0, 0, 0);
  }

  // Main loop over K tiles; LDS buffer `cur` holds tile it, the staging
  // registers tile it+1.
  for (int it = it0; it < it1; ++it) {
    const int cur = (it - it0) & 1, nxt = cur ^ 1;
    substep(std::integral_constant<int, 0>{}, cur, nxt);
    substep(std::integral_constant<int, 1>{}, cur, nxt);
    substep(std::integral_constant<int, 2>{}, cur, nxt);   // + stores of tile it+1 -> nxt
    __syncthreads();
    set_tiles(it + 2);
    substep(std::integral_constant<int, 3>{}, nxt, nxt);   // + loads of tile it+2
  }
  __syncthreads();  // the epilogue reuses LDS

  // Epilogue.  acc[i][j][4q + e] holds C[m][n + e] with
  //   m = m0 + wm*WTM + i*32 + (lane & 31),  n = n0 + wn*WTN + j*32 + 8q + 4*(lane >> 5).
  // One 32-row block per pass is staged through LDS (rows padded by 4 floats so
  // the 16-byte writes of 16 consecutive rows hit distinct banks); each wave then
  // walks its own block row-major, 4 columns per lane, through one rolled copy of
  // the epilogue: coalesced C accesses and no per-fragment epilogue code.
  constexpr int PITCH = WTN + 4;
  float* stg = reinterpret_cast<float*>(&smem[0][0]) + wave * (32 * PITCH);
  float* W = (p.splits > 1) ? p.ws + ((int64_t)tc.z * p.splits + tc.split) * (int64_t)p.M * p.N
                            : nullptr;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4_t v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (MODE == MODE_DUAL)
            v[e] = silu_f(p.alpha * acc[i][j][4 * q + e]) * (p.alpha * acc[i][j + TN][4 * q + e]);
          else
            v[e] = acc[i][j][4 * q + e];
        }
        *reinterpret_cast<f32x4_t*>(stg + lrow * PITCH + j * 32 + 8 * q + 4 * lhalf) = v;
      }
    __syncthreads();
    const int mrow0 = m0 + wm * WTM + i * 32;
    const int ncol0 = n0 + wn * WTN;
#pragma unroll 2
    for (int idx = lane; idx < 32 * (WTN / 4); idx += 64) {
      const int r = idx / (WTN / 4), c4 = idx - r * (WTN / 4);
      const f32x4_t sv = *reinterpret_cast<const f32x4_t*>(stg + r * PITCH + c4 * 4);
      const int m = mrow0 + r, n = ncol0 + c4 * 4;
      if (W) {
        if (m < p.M) {
          // partial slabs are 16-byte aligned (the workspace is; M*N*4 per slab)
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
        for (int e = 0; e < 4; ++e) v[e] = (MODE == MODE_DUAL) ? sv[e] : p.alpha * sv[e];
        epilogue4(p, Cz, Rz, m, n, v);
      }
    }
    __syncthreads();
  }
}

}  // namespace mig
