// mi_gemm.hip -- host dispatch and C ABI of the gfx950 GEMM core (include/mi_gemm.h).
//
// Replaces the GEMM entry points of the reference engine's Metal bridge
// (metal_bridge::gemm_bf16 / gemm_backward / gemm_proj_trans_b / gemm_proj /
// gemm_ffn / fused_swiglu_gemm, MetalBridge.hpp:39-46,119-125) and the batched
// branch of Tensor::matmul (Tensor.cpp:196-227).  Arguments are validated on the
// host and reported as status codes (the reference bridge printed and returned,
// MetalBridge.mm:1360; Tensor::matmul threw, Tensor.cpp:175-205 -- the C++ and
// Python mirrors above this ABI restore those behaviours).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/mi_gemm.h"
#include "mi_attn.hpp"
#include "mi_xent.hpp"
#include "mi_norm.hpp"
#include "mi_convert.hpp"
#include "mi_gemm_kernels.hpp"

using namespace mig;

// Split-K scratch of mi_gemm_noalloc: a file-scope device array, one copy per GPU
// the library runs on, held until the process ends.  Host code never passes the
// array's name to a kernel or copy (on the host it only stands in for the symbol):
// its device address is looked up once per device with hipGetSymbolAddress
// (scratch_of_current) and that address is what the kernels receive.
static __device__ __align__(256) float scratch[MI_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

struct DeviceInfo {
  bool ok = false;
  int cus = 256;
};
std::once_flag g_once;
DeviceInfo g_dev[64];
int g_init_status = MI_ERR_NO_DEVICE;

int init_devices() {
  std::call_once(g_once, [] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
      g_init_status = MI_ERR_NO_DEVICE;
      return;
    }
    bool any = false;
    for (int d = 0; d < n && d < 64; ++d) {
      hipDeviceProp_t prop;
      if (hipGetDeviceProperties(&prop, d) != hipSuccess) continue;
      if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) continue;
      g_dev[d].ok = true;
      g_dev[d].cus = prop.multiProcessorCount;
      any = true;
    }
    g_init_status = any ? MI_OK : MI_ERR_NO_DEVICE;
  });
  if (g_init_status != MI_OK) return fail(g_init_status, "no gfx950 device visible");
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64 || !g_dev[d].ok)
    return fail(MI_ERR_NO_DEVICE, "current device %d is not a gfx950", d);
  return MI_OK;
}

constexpr size_t kScratchBytes = MI_NOALLOC_SCRATCH_BYTES;
std::mutex g_scratch_mu;
void* g_scratch_ptr[64];

// Device address of `scratch` on the current device (looked up on first use).
int scratch_of_current(void** out) {
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64)
    return fail(MI_ERR_NO_DEVICE, "no current device");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[d]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(MI_ERR_HIP, "scratch symbol address on device %d: %s", d, hipGetErrorString(e));
    g_scratch_ptr[d] = ptr;
  }
  *out = g_scratch_ptr[d];
  return MI_OK;
}

int current_cus() {
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess) return 256;
  return (d >= 0 && d < 64 && g_dev[d].ok) ? g_dev[d].cus : 256;
}

// ---- kernel table ------------------------------------------------------------

KernelFn pick_kernel(int dtype_in, int transA, int transB, int cfg, bool fast, bool ktail,
                     int fast_epi) {
  const int lay = (transA ? 2 : 0) | (transB ? 1 : 0);
  if (dtype_in == MI_BF16) {
    switch (lay) {
      case 0: return pick_bf16_00(cfg, fast, ktail, fast_epi);
      case 1: return pick_bf16_01(cfg, fast, ktail, fast_epi);
      case 2: return pick_bf16_10(cfg, fast, ktail, fast_epi);
      default: return pick_bf16_11(cfg, fast, ktail, fast_epi);
    }
  }
  switch (lay) {
    case 0: return pick_f32_00(cfg, fast, ktail, fast_epi);
    case 1: return pick_f32_01(cfg, fast, ktail, fast_epi);
    case 2: return pick_f32_10(cfg, fast, ktail, fast_epi);
    default: return pick_f32_11(cfg, fast, ktail, fast_epi);
  }
}

CfgShape shape_of(int dtype_in, int cfg) { return cfg_shape(dtype_in == MI_BF16, cfg); }

// Split-K reduction: C = epilogue(alpha * sum_s ws[z][s]) in fixed split order.
__global__ void __launch_bounds__(256) splitk_reduce_kernel(Params p) {
  const int64_t per_z = (int64_t)p.M * ((p.N + 3) / 4);
  const int64_t total = per_z * p.batch;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * 256) {
    const int z = (int)(idx / per_z);
    const int64_t r = idx - (int64_t)z * per_z;
    const int m = (int)(r / ((p.N + 3) / 4));
    const int n = (int)(r - (int64_t)m * ((p.N + 3) / 4)) * 4;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    const bool vec = (p.N & 3) == 0;  // whole, 16-byte aligned quads of the partial slabs
    const float* W0 = p.ws + (int64_t)z * p.splits * (int64_t)p.M * p.N + (int64_t)m * p.N + n;
    const int64_t slab = (int64_t)p.M * p.N;
    if (vec) {
      // all splits' loads issued before the sum, which keeps the fixed split order
      for (int s = 0; s < p.splits; s += 8) {
        f32x4_t w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          w[u] = s + u < p.splits ? *(const f32x4_t*)(W0 + (s + u) * slab) : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (s + u < p.splits)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += w[u][e];
      }
    } else {
      for (int s = 0; s < p.splits; ++s) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < p.N) v[e] += W0[s * slab + e];
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] *= p.alpha;
    const int zo = z / p.heads, zi = z - (z / p.heads) * p.heads;
    const int64_t coff = (int64_t)zo * p.cO + (int64_t)(zi / p.gC) * p.cI;
    void* Cz = (char*)p.C + coff * (p.c_bf16 ? 2 : 4);
    const void* Rz = p.R ? (const char*)p.R + ((int64_t)zo * p.rO + (int64_t)zi * p.rI) * (p.r_bf16 ? 2 : 4)
                         : nullptr;
    epilogue4(p, Cz, Rz, m, n, v);
  }
}

// act[m, k] = SiLU(G[m, k]) * U[m, k] for the SiLU-gate prologue run as its own
// pass (bf16, 8 elements per thread, K a multiple of 8; G and U share the
// leading dimension ld, act is packed with leading dimension K).  The same
// arithmetic as the in-load prologue (swiglu_chunk): fp32, rounded to bf16.
__global__ void __launch_bounds__(256) swiglu_act_kernel(const __bf16* G, const __bf16* U, int64_t ld,
                                                         int64_t M, int64_t K, __bf16* act) {
  const int64_t cpr = K / 8;  // 16-byte chunks per row
  const int64_t n = M * cpr;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / cpr, c = i - m * cpr;
    const u32x4_t g = *(const u32x4_t*)(G + m * ld + c * 8);
    const u32x4_t u = *(const u32x4_t*)(U + m * ld + c * 8);
    *(u32x4_t*)(act + m * K + c * 8) = swiglu_chunk<__bf16>(g, u);
  }
}

// ---- planning ------------------------------------------------------------------

struct Plan {
  int cfg;
  int splits;
  int tiles_m, tiles_n;
};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Tile and split choice.  Rules fitted to forced-plan sweeps of the decoder-block
// and LM-head shapes on MI355X (TFLOP/s of bf16 256x256 "L" vs 128x128 "S" tiles,
// split-K factor after the letter):
//   * a grid of L tiles covering the CUs at least once runs as is (8192x2048x
//     5632 NT: L1 1375 vs S1 1180; 8192x32000x2048: L1 1256 vs S1 978), unless
//     its last wave is at most half full and S tiles fill whole waves
//     (8192x3072x2048: S1 1063 vs L1 1016);
//   * L tiles that leave a quarter of their area empty (N or M well below a
//     multiple of 256) use S;
//   * bf16 below one wave of L tiles: S tiles, two workgroups per CU, without
//     split (2048x2048x8192: S1 967 vs L2 640, S2 754; 2048x3072x8192: S1 887
//     vs L2 836).  With inputs and an fp32 beta = 1 output cold in HBM, as in
//     a training step, S also beats L1 on 2048x5632x8192 (931-951 vs 913): the
//     second workgroup on a CU hides the first one's C read-modify-write, which
//     L tiles all do at once (in a hot-cache loop L1 leads, 1143 vs 1038);
//   * when even S tiles leave half the CUs idle, K is split over S tiles, given
//     a workspace -- also for S tiles chosen by the fill rule and for the
//     register-staged loader (unaligned operands);
//   * fp32: 64x128 or 64x64 direct-to-LDS tiles with K split to about three
//     units per CU (16-byte-aligned operands), 128x128 register-staged tiles
//     split below 5/8 of a wave (element-granular loader); the rules at the fp32
//     branch.
// Every split fits the workspace: splits * M * N * batch <= ws_limit_elems.
Plan make_plan(int dtype_in, int64_t M, int64_t N, int64_t Ktot, int64_t batch, int mode,
               bool allow_split, int64_t ws_limit_elems, int cus, bool fast) {
  auto plan_for = [&](int cfg, int sp) {
    const CfgShape s = shape_of(dtype_in, cfg);
    return Plan{cfg, sp, (int)cdiv(M, s.bm), (int)cdiv(N, s.bn)};
  };
  if (mode == MODE_DUAL) return plan_for(CFG_DUAL, 1);
  if (mode == MODE_PROLOGUE) return plan_for(CFG_PRO, 1);
  const CfgShape L = shape_of(dtype_in, CFG_L), S = shape_of(dtype_in, CFG_S);
  const int64_t tilesL = cdiv(M, L.bm) * cdiv(N, L.bn) * batch;
  const int64_t tilesS = cdiv(M, S.bm) * cdiv(N, S.bn) * batch;
  const double fillL = (double)(M * N * batch) / ((double)tilesL * L.bm * L.bn);
  const double fillS = (double)(M * N * batch) / ((double)tilesS * S.bm * S.bn);
  // split K until the units cover the CUs once; each split keeps >= 8 K tiles
  // of 32 and its partials fit the workspace
  auto split_of = [&](int64_t tiles, int kt) {
    int sp = (int)std::min<int64_t>(cus / std::max<int64_t>(tiles, 1), 8);
    while (sp > 1 && (cdiv(Ktot, kt) < 8 * sp || (int64_t)sp * M * N * batch > ws_limit_elems)) --sp;
    return sp;
  };
  if (dtype_in == MI_BF16) {
    const bool sparse_L = fillL < 0.75 && fillS > fillL;
    if (fast && !sparse_L && tilesL >= cus) {
      const double waves = (double)tilesL / cus;
      const double frac = waves - std::floor(waves);
      // 256x192 tiles when they fill whole rounds where 256x256 tiles leave a
      // partial one (8192x3072x2048 NN: 94 us vs 103 for S, 108 for L)
      const int64_t tilesM = cdiv(M, 256) * cdiv(N, 192) * batch;
      if (frac > 0.0 && N % 192 == 0 && tilesM % cus == 0) return plan_for(CFG_M, 1);
      if (frac > 0.0 && frac <= 0.5 && tilesS >= cus) return plan_for(CFG_S, 1);
      return plan_for(CFG_L, 1);
    }
    // Below one wave of L tiles (long K): one partial round of L tiles or of 256x192
    // tiles (M), 128x128 tiles two 4-wave workgroups per CU (S), or one 8-wave
    // workgroup per CU that splits every K tile between two wave groups (W,
    // wave-level split-K).  Cost in units of one W tile, measured on the dW shapes
    // at K = 8192: an L tile (4x the work) takes 2.6, an M tile 3/4 of that, S tiles
    // 1.8 per round of two per CU and 1.1 alone (2048x5632: M 167 us (240 tiles), L
    // 177 (176), W 184, S 189; 5632x2048: M 164, L 172; 2048x3072: S 123, M 130, L
    // 165; 2048x2048: W 69, S 73, M 135, L 153).  M needs N in 64-column blocks.
    if (tilesS * 2 >= cus || !allow_split) {
      if (fast && !sparse_L && Ktot >= 1024) {
        const double cW = (double)cdiv(tilesS, cus);
        const int64_t full2 = tilesS / (2 * cus), rem = tilesS - full2 * 2 * cus;
        const double cS = 1.8 * (double)full2 + (rem > cus ? 1.8 : rem > 0 ? 1.1 : 0.0);
        const double cL = 2.6 * (double)cdiv(tilesL, cus);
        const int64_t tilesM = cdiv(M, 256) * cdiv(N, 192) * batch;
        const double cM = N % 64 == 0 ? 1.95 * (double)cdiv(tilesM, cus) : 1e30;
        // 128x192 split-K tiles (V): 1.5 W tiles of work, one workgroup per CU
        const int64_t tilesV = cdiv(M, 128) * cdiv(N, 192) * batch;
        const double cV = N % 64 == 0 ? 1.5 * (double)cdiv(tilesV, cus) : 1e30;
        if (cV < cM && cV < cL && cV < cW && cV < cS) return plan_for(CFG_V, 1);
        if (cM < cL && cM <= cW && cM <= cS) return plan_for(CFG_M, 1);
        if (cL <= cW && cL <= cS) return plan_for(CFG_L, 1);
        if (cW < cS) return plan_for(CFG_W, 1);
      }
      return plan_for(CFG_S, 1);
    }
    return plan_for(CFG_S, split_of(tilesS, 32));
  }
  // fp32 with the direct-to-LDS kernel: 64x128 tiles (V; four waves of 32x64) or 64x64
  // tiles (M; four waves of 32x32), several workgroups per CU.  Score of a plan: the
  // busiest CU's share of the work, ceil(units / cus) x tile area / splits (units =
  // tiles x splits, at most three per CU once split, each split keeping at least 512 of
  // K, or 128 while the units fit one per CU: configuration 1, 48 tiles at K = 768,
  // splits 5).  Lowest score; ties to fewer splits, then to 64x128 tiles when K < 1024
  // and 64x64 tiles otherwise.  Fitted to a forced-plan sweep of configuration 2's 12
  // distinct GEMMs over these tiles, 128x128, and splits 1..8 (hot loop, TFLOP/s):
  // qkv forward 2048x2304x768 64x64 115 vs 64x128 92; 2048x768x2048 (gate / qkv dX,
  // down forward, down / gate dW) 64x64 split 2 113-117 vs 64x128 split 4 104-109;
  // qkv dW 768x2304x2048 64x64 113 vs 64x128 102; o forward 2048x768x768 64x128 93 vs
  // 64x64 87; gate forward 2048x2048x768 64x128 127 vs 64x64 122.  The rule picks the
  // best plan of every one of the 12, or one within 2 %.
  // The element-granular loader (any alignment) runs 128x128 tiles (S): below 5/8
  // of a wave, K is split by the same score with units at most two per CU and each
  // split keeping >= 8 K tiles of 32, or >= 4 when the units fit one per CU (96
  // tiles at K = 2048: splits 1..8 ran 43 71 59 74 83 66 69 76 TFLOP/s; 108 tiles:
  // 47 78 67 83 65 73 76 71; 36 tiles: 16 28 37 44 49 52 54 41).
  if (fast) {
    int best_cfg = CFG_V, best_sp = 1;
    double best_score = 1e300;
    for (int cfg : {CFG_V, CFG_M}) {
      const CfgShape t = shape_of(dtype_in, cfg);
      const int64_t tiles = cdiv(M, t.bm) * cdiv(N, t.bn) * batch;
      for (int sp = 1; sp <= (allow_split ? 8 : 1); ++sp) {
        const int64_t units = tiles * sp;
        if (sp > 1) {
          if (units > 3 * (int64_t)cus || (int64_t)sp * M * N * batch > ws_limit_elems) continue;
          if (Ktot < (units > cus ? 512 : 128) * (int64_t)sp) continue;
        }
        const double score = (double)cdiv(units, cus) * t.bm * t.bn / sp;
        const bool wins = score < best_score ||
                          (score == best_score &&
                           (sp < best_sp || (sp == best_sp && cfg == (Ktot < 1024 ? CFG_V : CFG_M))));
        if (wins) best_cfg = cfg, best_sp = sp, best_score = score;
      }
    }
    return plan_for(best_cfg, best_sp);
  }
  if (tilesS * 8 >= (int64_t)cus * 5 || !allow_split) return plan_for(CFG_S, 1);
  const int64_t kts = cdiv(Ktot, 32);
  int best = 1;
  double best_score = 1.0;
  for (int sp = 2; sp <= 8; ++sp) {
    const int64_t units = tilesS * sp;
    if (units > 2 * (int64_t)cus || (int64_t)sp * M * N * batch > ws_limit_elems) continue;
    if (cdiv(kts, sp) < (units <= cus ? 4 : 8)) continue;
    const double score = (double)cdiv(units, cus) / sp;
    if (score <= best_score) best = sp, best_score = score;
  }
  return plan_for(CFG_S, best);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Text of a plan, as mi_gemm_describe and the profiler records show it.
void describe_plan(char* buf, size_t len, int dtype_in, bool fast, const Plan& pl, int transA,
                   int transB, int64_t batch) {
  const CfgShape sh = shape_of(dtype_in, pl.cfg);
  const char* kind = (dtype_in == MI_BF16 && fast && pl.cfg != CFG_PRO)
                         ? (pl.cfg == CFG_W || pl.cfg == CFG_V ? "dlds-kg2" : "dlds")
                     : (dtype_in != MI_BF16 && fast && (pl.cfg == CFG_V || pl.cfg == CFG_M)) ? "dlds"
                                                                                           : "regstage";
  std::snprintf(buf, len, "%s %s %dx%d %s%s split%d tiles%lld", kind,
                dtype_in == MI_BF16 ? "bf16" : "f32", sh.bm, sh.bn, transA ? "T" : "N",
                transB ? "T" : "N", pl.splits, (long long)pl.tiles_m * pl.tiles_n * batch);
}

// ---- per-call GEMM profiler ----------------------------------------------------
// When enabled, run() brackets each problem's launches (the GEMM and its split-K
// reduction) with two HIP events on the caller's stream and keeps a record of the
// problem, its plan and the events; the elapsed time is read when a record is
// asked for.  Events are recycled per device.
struct ProfEntry {
  mi_gemm_record rec;
  hipEvent_t e0, e1;
  int dev;
  bool resolved;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<ProfEntry> g_prof;
std::vector<hipEvent_t> g_prof_free[64];
double g_prof_total_ms = 0.0;
int64_t g_prof_calls = 0;

hipEvent_t prof_event(int dev) {
  if (!g_prof_free[dev].empty()) {
    hipEvent_t e = g_prof_free[dev].back();
    g_prof_free[dev].pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  return hipEventCreate(&e) == hipSuccess ? e : nullptr;
}

// Wait for entry i's events and add its time to the totals (once).
int prof_resolve(ProfEntry& en) {
  if (en.resolved) return MI_OK;
  float ms = 0.0f;
  if (hipEventSynchronize(en.e1) != hipSuccess || hipEventElapsedTime(&ms, en.e0, en.e1) != hipSuccess)
    return fail(MI_ERR_HIP, "profiler: event wait failed");
  en.rec.gpu_ms = ms;
  en.resolved = true;
  g_prof_total_ms += ms;
  g_prof_calls += 1;
  return MI_OK;
}

// Two row arrays of `bytes` bytes each that share memory without being the same array.
bool rows_overlap(const void* a, const void* b, int64_t bytes) {
  if (!a || !b || a == b) return false;
  const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
  return a0 < b0 + (uintptr_t)bytes && b0 < a0 + (uintptr_t)bytes;
}

struct Problem {
  int transA, transB;
  int64_t M, N, K;
  float alpha, beta;
  const void *A, *B;
  int64_t lda, ldb;
  int dtype_in;
  void* C;
  int64_t ldc;
  int dtype_c;
  mi_batch bt;
  mi_epilogue ep;
  void* ws;
  size_t ws_bytes;
  bool noalloc = false;  // mi_gemm_noalloc: the library's static scratch is the workspace
};

int validate(const Problem& P) {
  if (P.M < 0 || P.N < 0 || P.K < 0) return fail(MI_ERR_SHAPE, "negative size M=%lld N=%lld K=%lld",
                                                 (long long)P.M, (long long)P.N, (long long)P.K);
  if (P.M > INT32_MAX || P.N > INT32_MAX || P.K > INT32_MAX)
    return fail(MI_ERR_SHAPE, "size exceeds 2^31-1");
  if (P.dtype_in != MI_F32 && P.dtype_in != MI_BF16)
    return fail(MI_ERR_DTYPE, "input dtype %d not supported", P.dtype_in);
  if (P.dtype_c != MI_F32 && P.dtype_c != MI_BF16)
    return fail(MI_ERR_DTYPE, "output dtype %d not supported", P.dtype_c);
  if (P.M == 0 || P.N == 0) return MI_OK;
  if (!P.C) return fail(MI_ERR_NULL, "C is NULL");
  if (P.ldc < P.N) return fail(MI_ERR_LD, "ldc=%lld < N=%lld", (long long)P.ldc, (long long)P.N);
  if (P.K > 0) {
    if (!P.A || !P.B) return fail(MI_ERR_NULL, "A or B is NULL");
    const int64_t a_row = P.transA ? P.M : P.K, b_row = P.transB ? P.K : P.N;
    if (P.lda < a_row) return fail(MI_ERR_LD, "lda=%lld < %lld", (long long)P.lda, (long long)a_row);
    if (P.ldb < b_row) return fail(MI_ERR_LD, "ldb=%lld < %lld", (long long)P.ldb, (long long)b_row);
  }
  const mi_batch& b = P.bt;
  if (b.batch < 1 || b.heads < 1 || b.a_group < 1 || b.b_group < 1 || b.c_group < 1 ||
      b.k_segments < 1)
    return fail(MI_ERR_SHAPE, "batch, heads, groups and k_segments must be >= 1");
  if (b.batch > 65535LL * 1024) return fail(MI_ERR_SHAPE, "batch too large");
  if (b.causal < MI_CAUSAL_NONE || b.causal > MI_CAUSAL_A_UPPER)
    return fail(MI_ERR_SHAPE, "unknown causal mode %d", b.causal);
  if (b.k_segments * P.K > INT32_MAX) return fail(MI_ERR_SHAPE, "total K exceeds 2^31-1");
  const mi_epilogue& e = P.ep;
  if (e.A2 && e.B2) return fail(MI_ERR_UNSUPPORTED, "A2 prologue and B2 dual-B cannot be combined");
  if (e.A2 && P.transA) return fail(MI_ERR_UNSUPPORTED, "SiLU-gate prologue needs transA = 0");
  if (e.residual && e.ldr < P.N) return fail(MI_ERR_LD, "ldr=%lld < N", (long long)e.ldr);
  if (e.bias && e.bias_dtype != MI_F32 && e.bias_dtype != MI_BF16)
    return fail(MI_ERR_DTYPE, "bias dtype %d", e.bias_dtype);
  if (e.residual && e.residual_dtype != MI_F32 && e.residual_dtype != MI_BF16)
    return fail(MI_ERR_DTYPE, "residual dtype %d", e.residual_dtype);
  if (e.B2 && b.causal == MI_CAUSAL_OUT_LOWER)
    return fail(MI_ERR_UNSUPPORTED, "dual-B with causal output mask");
  if (e.row_scale && (e.B2 || b.batch != 1))
    return fail(MI_ERR_UNSUPPORTED, "row_scale needs one problem without dual-B");
  if (e.row_scale && ((uintptr_t)e.row_scale & 3u))
    return fail(MI_ERR_UNSUPPORTED, "row_scale must be 4-byte aligned");
  return MI_OK;
}

// Tile rows per column sweep of the tile order (group_m of map_tile).  The tiles
// an XCD holds at once share their A and B panels in that XCD's L2, which fetches
// each panel's K rows once per K step; fewer distinct panels per XCD means fewer
// L2 fills.  For one bf16 problem without split-K, the host walks map_tile's order
// for each XCD's resident tiles (its first round: 32 CUs x workgroups per CU)
// and takes the group height in {1, 2, 4, 8, 16} whose XCDs fill the fewest panel
// bytes, sum over XCDs of (distinct row panels x BM + distinct column panels x BN)
// per K row.  For bf16 C, ties go to the height whose resident tiles span more
// column panels, then to 8 (fp32 C: to 8): the C tiles an XCD stores at once then
// cover a wider window of each output row.  With a row pitch that is a multiple of
// 4 KB (N = 2048 bf16), a window of 4 of the 8 column tiles (height 8) puts every
// row's stores in the same half of each 4 KB period, where the memory channels
// interleave; the full width (height 4, the same panel bytes) measured 1092 -> 1146
// TFLOP/s (o projection, 8192 x 2048 x 2048 forward), 1111 -> 1180 (its dX), 1210
// -> 1264 (QKV dX) and 1325 -> 1361 (down forward), alternating on one box; a
// padded C pitch (+128 bytes) gave the same gains with height 8.  The fp32 weight
// gradients do not gain: the o projection's (2048 x 2048, 128 x 128 tiles) lost
// 3.6 % in the block set with the wider window.  Configuration 3's 2048 x 5632
// weight gradients (240 tiles of 256 x 192, 30 per XCD) get 4 (4 row panels x 7.5
// column panels: 2464 panel columns per K row against 2768 for 8 x 3.75); block
// set with per-XCD K rotation 1110-1114 -> 1126-1128 TFLOP/s on one box (gate dW
// 917-926 -> 1022-1036).
int group_rows(const Problem& P, const Plan& plan) {
  const mi_batch& b = P.bt;
  if (P.dtype_in != MI_BF16 || plan.splits != 1 || b.batch != 1 || b.causal != MI_CAUSAL_NONE)
    return MI_GROUP_M;
  const CfgShape ts = shape_of(P.dtype_in, plan.cfg);
  const int64_t tm = plan.tiles_m, tn = plan.tiles_n, tiles = tm * tn;
  const int per_cu = ts.threads >= 512 ? 1 : 2;
  const int64_t resident = std::max<int64_t>(1, (int64_t)current_cus() / 8 * per_cu);
  const int64_t q = tiles / 8, rem = tiles % 8;
  int best = MI_GROUP_M;
  int64_t best_cost = INT64_MAX, best_cols = 0;
  std::vector<char> seen_m((size_t)tm), seen_n((size_t)tn);
  for (int g : {8, 16, 4, 2, 1}) {
    int64_t cost = 0, cols = 0;
    for (int64_t x = 0; x < 8; ++x) {
      const int64_t first = x * q + std::min<int64_t>(x, rem);
      const int64_t count = std::min<int64_t>(q + (x < rem ? 1 : 0), resident);
      std::fill(seen_m.begin(), seen_m.end(), 0);
      std::fill(seen_n.begin(), seen_n.end(), 0);
      int64_t dm = 0, dn = 0;
      for (int64_t t = first; t < first + count; ++t) {
        // map_tile's order (mi_gemm_device.hpp) for logical tile t
        const int64_t group = (int64_t)g * tn, gi = t / group, first_m = gi * g;
        const int64_t gm = std::min<int64_t>(tm - first_m, g), r = t - gi * group;
        const int64_t m = first_m + r % gm, n = r / gm;
        if (!seen_m[(size_t)m]) seen_m[(size_t)m] = 1, ++dm;
        if (!seen_n[(size_t)n]) seen_n[(size_t)n] = 1, ++dn;
      }
      cost += dm * ts.bm + dn * ts.bn;
      cols += dn;
    }
    const bool wider = P.dtype_c == MI_BF16 && cols > best_cols;
    if (cost < best_cost || (cost == best_cost && wider)) best_cost = cost, best_cols = cols, best = g;
  }
  return best;
}

// Operand layouts whose GEMMs rotate K per XCD.
bool rotate_policy(int transA, int transB) {
  (void)transA; (void)transB;
  return true;
}

// Per-XCD K rotation of the direct-to-LDS kernels (see gemm_dlds_kernel): one
// problem, one K segment, no split-K, no causal skipping.
bool rotate_k(const Problem& P, const Plan& plan) {
  const mi_batch& b = P.bt;
  if (P.dtype_in != MI_BF16 || plan.splits != 1 || b.batch != 1 || b.k_segments != 1 ||
      b.causal != MI_CAUSAL_NONE || plan.cfg == CFG_PRO)
    return false;
  return rotate_policy(P.transA, P.transB);
}

int run(const Problem& P, hipStream_t stream) {
  int st = validate(P);
  if (st != MI_OK) return st;
  if (P.M == 0 || P.N == 0) return MI_OK;
  st = init_devices();
  if (st != MI_OK) return st;

  const int mode = P.ep.B2 ? MODE_DUAL : (P.ep.A2 ? MODE_PROLOGUE : MODE_PLAIN);
  const int CH = P.dtype_in == MI_BF16 ? 8 : 4;
  const mi_batch& b = P.bt;

  // 16-byte operand loads need every chunk start 16-byte aligned.
  auto mult = [&](int64_t v) { return v % CH == 0; };
  const bool vecA = aligned16(P.A) && (!P.ep.A2 || aligned16(P.ep.A2)) && mult(P.lda) &&
                    mult(b.a_outer) && mult(b.a_inner) && mult(b.seg_a);
  const bool vecB = aligned16(P.B) && (!P.ep.B2 || aligned16(P.ep.B2)) && mult(P.ldb) &&
                    mult(b.b_outer) && mult(b.b_inner) && mult(b.seg_b);
  const int ce = P.dtype_c == MI_BF16 ? 8 : 16;  // bytes of 4 C elements
  auto al = [](const void* p, int a) { return ((uintptr_t)p % a) == 0; };
  const bool cvec = al(P.C, ce) && P.ldc % 4 == 0 && b.c_outer % 4 == 0 && b.c_inner % 4 == 0 &&
                    (!P.ep.bias || al(P.ep.bias, P.ep.bias_dtype == MI_BF16 ? 8 : 16)) &&
                    (!P.ep.residual || (al(P.ep.residual, P.ep.residual_dtype == MI_BF16 ? 8 : 16) &&
                                        P.ep.ldr % 4 == 0 && b.r_outer % 4 == 0 && b.r_inner % 4 == 0));

  // Fast (buffer-load) path: chunks never straddle a matrix edge and every byte
  // offset the loaders form stays below 2^31.
  const int esz = P.dtype_in == MI_BF16 ? 2 : 4;
  const int64_t a_rows = P.M, b_rows = P.N;
  const int64_t a_contig = P.transA ? P.M : P.K, b_contig = P.transB ? P.K : P.N;
  const int64_t extA = P.K == 0 ? 0 : (P.transA ? (P.K - 1) * P.lda + P.M : (P.M - 1) * P.lda + P.K) * esz;
  const int64_t extB = P.K == 0 ? 0 : (P.transB ? (P.N - 1) * P.ldb + P.K : (P.K - 1) * P.ldb + P.N) * esz;
  const int64_t lim = (int64_t)1 << 31;
  auto span_ok = [&](bool kc, int64_t rows, int64_t ld) {
    // largest offset formed: a row/k line one tile (<= 512 rows, <= 64 k) past the edge
    const int64_t far = kc ? (rows + 512) * ld * esz + (P.K + 64) * esz
                           : (P.K + 64) * ld * esz + (rows + 512) * esz;
    return far < lim;
  };
  const bool fast = vecA && vecB && mult(a_contig) && mult(b_contig) && extA < lim && extB < lim &&
                    span_ok(!P.transA, a_rows, P.lda) && span_ok(P.transB != 0, b_rows, P.ldb);

  // SiLU-gate prologue as its own pass when the workspace holds SiLU(A) * A2 (bf16,
  // one matrix, 16-byte rows): the activation is written once and the GEMM runs
  // the direct-to-LDS kernel on it, where the in-load prologue would recompute it
  // for every column tile in the register-staged loader (configuration 3's down
  // projection 8192x2048x5632: 426 us in-load vs about 210 us in two passes).
  // mi_gemm_noalloc never takes it: its fixed scratch is sized for split-K partials,
  // not for an M x K activation, so it runs the in-load prologue (the plan mi_gemm
  // makes without a workspace).
  if (mode == MODE_PROLOGUE && !P.noalloc && P.dtype_in == MI_BF16 && !P.transA && P.K > 0 &&
      b.batch == 1 &&
      b.k_segments == 1 && vecA && P.K % 8 == 0 && aligned16(P.ws) &&
      P.ws_bytes >= (size_t)(P.M * P.K * 2)) {
    const size_t act_bytes = (size_t)((P.M * P.K * 2 + 255) / 256 * 256);
    __bf16* act = (__bf16*)P.ws;
    const int64_t chunks = P.M * (P.K / 8);
    const int64_t grid = std::min<int64_t>(cdiv(chunks, 256), 8 * (int64_t)current_cus());
    hipLaunchKernelGGL(swiglu_act_kernel, dim3((unsigned)grid), dim3(256), 0, stream, (const __bf16*)P.A,
                       (const __bf16*)P.ep.A2, P.lda, P.M, P.K, act);
    const hipError_t ea = hipGetLastError();
    if (ea != hipSuccess) return fail(MI_ERR_HIP, "SiLU-gate pass launch: %s", hipGetErrorString(ea));
    Problem Q = P;
    Q.A = act;
    Q.lda = P.K;
    Q.ep.A2 = nullptr;
    Q.ws = P.ws_bytes > act_bytes ? (char*)P.ws + act_bytes : nullptr;
    Q.ws_bytes = P.ws_bytes > act_bytes ? P.ws_bytes - act_bytes : 0;
    return run(Q, stream);
  }

  const int64_t Ktot = P.K * b.k_segments;
  const int64_t ws_elems = P.ws ? (int64_t)(P.ws_bytes / sizeof(float)) : 0;
  const bool allow_split = ws_elems > 0 && aligned16(P.ws);
  // mi_gemm_noalloc: the plan mi_gemm makes with unlimited workspace, refused when
  // its partials would not fit the scratch array (so both entry points run the same
  // kernels on the same problem)
  Plan plan = make_plan(P.dtype_in, P.M, P.N, Ktot, b.batch, mode, allow_split || P.noalloc,
                        P.noalloc ? INT64_MAX / 8 : ws_elems, current_cus(), fast);
  if (P.noalloc && plan.splits > 1 && (int64_t)plan.splits * P.M * P.N * b.batch > ws_elems)
    return fail(MI_ERR_WORKSPACE,
                "mi_gemm_noalloc: split-K by %d needs %lld bytes of scratch, above its %lld-byte "
                "maximum (call mi_gemm with a workspace)",
                plan.splits, (long long)plan.splits * P.M * P.N * b.batch * 4, (long long)ws_elems * 4);

  // The planner only splits within the workspace; checked again here because
  // an undersized workspace would take out-of-bounds partial-sum writes.
  if (plan.splits > 1 && ((int64_t)plan.splits * P.M * P.N * b.batch > ws_elems || !allow_split))
    return fail(MI_ERR_WORKSPACE, "split-K by %d needs %lld floats of workspace, %lld given",
                plan.splits, (long long)plan.splits * P.M * P.N * b.batch, (long long)ws_elems);
  const CfgShape ts = shape_of(P.dtype_in, plan.cfg);
  // the direct epilogue works in whole 32x32 blocks (an edge tile skips those past M, N)
  const bool fast_epi = plan.splits == 1 && !P.ep.bias && !P.ep.residual && cvec &&
                        b.causal != MI_CAUSAL_OUT_LOWER && P.M % 32 == 0 && P.N % 32 == 0;
  const int64_t kstep = P.dtype_in != MI_BF16 ? 32 : plan.cfg == CFG_W || plan.cfg == CFG_V ? MI_W_BK : 64;
  // with a row scale the direct epilogue has a variant of its own (A K-contiguous on the
  // 256x256, 256x192 and 128x128 tiles); elsewhere the general epilogue applies it
  int epi_kind = fast_epi ? 1 : 0;
  if (P.ep.row_scale && fast_epi)
    epi_kind = (P.dtype_in == MI_BF16 && fast && !P.transA && P.K % kstep == 0 &&
                (plan.cfg == CFG_L || plan.cfg == CFG_M || plan.cfg == CFG_S)) ? 2 : 0;
  KernelFn fn = pick_kernel(P.dtype_in, P.transA, P.transB, plan.cfg, fast, P.K % kstep != 0, epi_kind);
  if (!fn) return fail(MI_ERR_UNSUPPORTED, "no kernel for this layout / mode");

  Params p;
  std::memset(&p, 0, sizeof(p));
  p.A = P.A;
  p.A2 = P.ep.A2;
  p.B = P.B;
  p.B2 = P.ep.B2;
  p.C = P.C;
  p.bias = P.ep.bias;
  p.R = P.ep.residual;
  p.row_scale = P.ep.row_scale;
  p.ws = (float*)P.ws;
  p.lda = P.lda;
  p.ldb = P.ldb;
  p.ldc = P.ldc;
  p.ldr = P.ep.ldr;
  p.segA = b.seg_a;
  p.segB = b.seg_b;
  p.aO = b.a_outer; p.aI = b.a_inner;
  p.bO = b.b_outer; p.bI = b.b_inner;
  p.cO = b.c_outer; p.cI = b.c_inner;
  p.rO = b.r_outer; p.rI = b.r_inner;
  p.M = (int)P.M;
  p.N = (int)P.N;
  p.K = (int)P.K;
  p.nseg = (int)b.k_segments;
  p.heads = (int)b.heads;
  p.gA = (int)b.a_group;
  p.gB = (int)b.b_group;
  p.gC = (int)b.c_group;
  p.tiles_m = plan.tiles_m;
  p.tiles_n = plan.tiles_n;
  p.splits = plan.splits;
  p.batch = (int)b.batch;
  p.causal = b.causal;
  p.mask_value = b.mask_value;
  p.alpha = P.alpha;
  p.beta = P.beta;
  p.c_bf16 = P.dtype_c == MI_BF16;
  p.bias_bf16 = P.ep.bias_dtype == MI_BF16;
  p.r_bf16 = P.ep.residual_dtype == MI_BF16;
  p.vecA = vecA;
  p.vecB = vecB;
  p.cvec = cvec;
  p.extA = (uint32_t)(fast ? extA : 0);
  p.extB = (uint32_t)(fast ? extB : 0);
  p.krot = rotate_k(P, plan) ? 1 : 0;
  p.group_m = group_rows(P, plan);

  const int64_t nblocks = (int64_t)plan.tiles_m * plan.tiles_n * plan.splits * b.batch;
  if (nblocks > INT32_MAX) return fail(MI_ERR_SHAPE, "too many tiles");

  // profiler: events around this problem's launches (never on the no-allocation path)
  std::unique_lock<std::mutex> prof_lock(g_prof_mu, std::defer_lock);
  ProfEntry pe;
  bool prof = false;
  if (!P.noalloc) {
    prof_lock.lock();
    if (g_prof_on && hipGetDevice(&pe.dev) == hipSuccess && pe.dev >= 0 && pe.dev < 64) {
      pe.e0 = prof_event(pe.dev);
      pe.e1 = prof_event(pe.dev);
      prof = pe.e0 && pe.e1 && hipEventRecord(pe.e0, stream) == hipSuccess;
    }
    if (!prof) prof_lock.unlock();
  }

  auto drop_events = [&]() {
    if (prof) {
      g_prof_free[pe.dev].push_back(pe.e0);
      g_prof_free[pe.dev].push_back(pe.e1);
    }
  };
  hipLaunchKernelGGL(fn, dim3((unsigned)nblocks), dim3((unsigned)ts.threads), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return drop_events(), fail(MI_ERR_HIP, "gemm launch: %s", hipGetErrorString(e));
  if (plan.splits > 1) {
    const int64_t work = b.batch * P.M * ((P.N + 3) / 4);
    const int64_t grid = std::min<int64_t>(cdiv(work, 256), 8 * (int64_t)current_cus());
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)grid), dim3(256), 0, stream, p);
    e = hipGetLastError();
    if (e != hipSuccess)
      return drop_events(), fail(MI_ERR_HIP, "split-K reduce launch: %s", hipGetErrorString(e));
  }
  if (prof && hipEventRecord(pe.e1, stream) != hipSuccess) {
    drop_events();
  } else if (prof) {
    std::memset(&pe.rec, 0, sizeof(pe.rec));
    pe.rec.M = P.M; pe.rec.N = P.N; pe.rec.K = P.K; pe.rec.batch = b.batch;
    pe.rec.transA = P.transA; pe.rec.transB = P.transB;
    pe.rec.dtype_in = P.dtype_in; pe.rec.dtype_c = P.dtype_c;
    pe.rec.splits = plan.splits;
    pe.rec.gpu_ms = -1.0;
    describe_plan(pe.rec.kernel, sizeof(pe.rec.kernel), P.dtype_in, fast, plan, P.transA, P.transB,
                  b.batch);
    pe.resolved = false;
    g_prof.push_back(pe);
  }
  return MI_OK;
}

mi_batch single_batch() {
  mi_batch b;
  std::memset(&b, 0, sizeof(b));
  b.batch = 1;
  b.heads = 1;
  b.a_group = b.b_group = b.c_group = 1;
  b.k_segments = 1;
  return b;
}

// ---- aux kernels -----------------------------------------------------------------

template <bool BF>
__device__ __forceinline__ float ldv(const void* p, int64_t i) {
  if constexpr (BF) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  else return ((const float*)p)[i];
}
template <bool BF>
__device__ __forceinline__ void stv(void* p, int64_t i, float v) {
  if constexpr (BF) ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16_rne(v);
  else ((float*)p)[i] = v;
}

template <bool BF>
__global__ void __launch_bounds__(256) residual_add_kernel(void* a, const void* b, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    stv<BF>(a, i, ldv<BF>(a, i) + ldv<BF>(b, i));
}

__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(v, o, 64);
    v = is_max ? fmaxf(v, w) : v + w;
  }
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < 4; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
  return r;
}

// One workgroup per row; row r is query position q = r % T.
template <bool BF>
__global__ void __launch_bounds__(256) softmax_causal_kernel(void* S, int64_t T, int64_t ld) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t q = row % T;
  const int64_t base = row * ld;
  float mx = -INFINITY;
  for (int64_t k = threadIdx.x; k <= q; k += 256) mx = fmaxf(mx, ldv<BF>(S, base + k));
  mx = block_reduce(mx, true, red);
  float sum = 0.f;
  for (int64_t k = threadIdx.x; k <= q; k += 256) sum += __expf(ldv<BF>(S, base + k) - mx);
  sum = block_reduce(sum, false, red);
  const float inv = 1.0f / sum;
  for (int64_t k = threadIdx.x; k < T; k += 256)
    stv<BF>(S, base + k, k <= q ? __expf(ldv<BF>(S, base + k) - mx) * inv : 0.0f);
}

template <bool BF>
__global__ void __launch_bounds__(256) softmax_bwd_kernel(const void* P, void* dP, int64_t T,
                                                          int64_t ld, float scale) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t base = row * ld;
  float s = 0.f;
  for (int64_t k = threadIdx.x; k < T; k += 256) s += ldv<BF>(P, base + k) * ldv<BF>(dP, base + k);
  s = block_reduce(s, false, red);
  for (int64_t k = threadIdx.x; k < T; k += 256) {
    const float p = ldv<BF>(P, base + k);
    stv<BF>(dP, base + k, p * (ldv<BF>(dP, base + k) - s) * scale);
  }
}

}  // namespace

// ---- C ABI -------------------------------------------------------------------------

extern "C" {

int mi_init(void) {
  const int st = init_devices();
  if (st != MI_OK) return st;
  void* ptr = nullptr;
  return scratch_of_current(&ptr);  // set-up of mi_gemm_noalloc's scratch on this device
}

const char* mi_last_error(void) { return g_err.c_str(); }

const char* mi_version(void) { return "mi_gemm 0.1 (gfx950)"; }

size_t mi_gemm_workspace_size(int transA, int transB, int64_t M, int64_t N, int64_t K,
                              int32_t dtype_in, int32_t dtype_c, int64_t batch) {
  (void)transA; (void)transB; (void)dtype_c;
  if (M <= 0 || N <= 0 || K <= 0 || batch <= 0) return 0;
  int cus = 256;
  if (init_devices() == MI_OK) cus = current_cus();
  const Plan pl = make_plan(dtype_in, M, N, K, batch, MODE_PLAIN, true, INT64_MAX / 8, cus, true);
  return pl.splits > 1 ? (size_t)pl.splits * (size_t)M * (size_t)N * (size_t)batch * sizeof(float) : 0;
}

int mi_gemm(void* stream, int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha,
            const void* A, int64_t lda, const void* B, int64_t ldb, int32_t dtype_in, float beta,
            void* C, int64_t ldc, int32_t dtype_c, const mi_epilogue* epi, void* workspace,
            size_t workspace_bytes) {
  Problem P;
  P.transA = transA;
  P.transB = transB;
  P.M = M; P.N = N; P.K = K;
  P.alpha = alpha; P.beta = beta;
  P.A = A; P.B = B; P.lda = lda; P.ldb = ldb;
  P.dtype_in = dtype_in;
  P.C = C; P.ldc = ldc; P.dtype_c = dtype_c;
  P.bt = single_batch();
  if (epi) P.ep = *epi;
  else std::memset(&P.ep, 0, sizeof(P.ep));
  P.ws = workspace;
  P.ws_bytes = workspace_bytes;
  return run(P, (hipStream_t)stream);
}

int mi_gemm_noalloc(void* stream, int transA, int transB, int64_t M, int64_t N, int64_t K,
                    float alpha, const void* A, int64_t lda, const void* B, int64_t ldb,
                    int32_t dtype_in, float beta, void* C, int64_t ldc, int32_t dtype_c,
                    const mi_epilogue* epi) {
  Problem P;
  P.transA = transA;
  P.transB = transB;
  P.M = M; P.N = N; P.K = K;
  P.alpha = alpha; P.beta = beta;
  P.A = A; P.B = B; P.lda = lda; P.ldb = ldb;
  P.dtype_in = dtype_in;
  P.C = C; P.ldc = ldc; P.dtype_c = dtype_c;
  P.bt = single_batch();
  if (epi) P.ep = *epi;
  else std::memset(&P.ep, 0, sizeof(P.ep));
  P.noalloc = true;
  P.ws = nullptr;
  P.ws_bytes = 0;
  int st = validate(P);
  if (st != MI_OK) return st;
  if (M == 0 || N == 0) return MI_OK;
  if ((st = init_devices()) != MI_OK) return st;
  if ((st = scratch_of_current(&P.ws)) != MI_OK) return st;
  P.ws_bytes = kScratchBytes;
  return run(P, (hipStream_t)stream);
}

int mi_gemm_batched(void* stream, int transA, int transB, int64_t M, int64_t N, int64_t K,
                    float alpha, const void* A, int64_t lda, const void* B, int64_t ldb,
                    int32_t dtype_in, float beta, void* C, int64_t ldc, int32_t dtype_c,
                    const mi_batch* batch, const mi_epilogue* epi, void* workspace,
                    size_t workspace_bytes) {
  if (!batch) return fail(MI_ERR_NULL, "batch descriptor is NULL");
  Problem P;
  P.transA = transA;
  P.transB = transB;
  P.M = M; P.N = N; P.K = K;
  P.alpha = alpha; P.beta = beta;
  P.A = A; P.B = B; P.lda = lda; P.ldb = ldb;
  P.dtype_in = dtype_in;
  P.C = C; P.ldc = ldc; P.dtype_c = dtype_c;
  P.bt = *batch;
  if (epi) P.ep = *epi;
  else std::memset(&P.ep, 0, sizeof(P.ep));
  P.ws = workspace;
  P.ws_bytes = workspace_bytes;
  return run(P, (hipStream_t)stream);
}

int mi_residual_add(void* stream, void* a, const void* b, int64_t n, int32_t dtype) {
  if (n < 0) return fail(MI_ERR_SHAPE, "negative n");
  if (n == 0) return MI_OK;
  if (!a || !b) return fail(MI_ERR_NULL, "a or b is NULL");
  if (dtype != MI_F32 && dtype != MI_BF16) return fail(MI_ERR_DTYPE, "dtype %d", dtype);
  int st = init_devices();
  if (st != MI_OK) return st;
  const int64_t grid = std::min<int64_t>(cdiv(n, 256), 16 * (int64_t)current_cus());
  if (dtype == MI_BF16)
    hipLaunchKernelGGL(residual_add_kernel<true>, dim3((unsigned)grid), dim3(256), 0,
                       (hipStream_t)stream, a, b, n);
  else
    hipLaunchKernelGGL(residual_add_kernel<false>, dim3((unsigned)grid), dim3(256), 0,
                       (hipStream_t)stream, a, b, n);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MI_OK : fail(MI_ERR_HIP, "residual_add: %s", hipGetErrorString(e));
}

int mi_softmax_causal(void* stream, void* S, int64_t rows, int64_t T, int64_t ld, int32_t dtype) {
  if (rows < 0 || T < 0) return fail(MI_ERR_SHAPE, "negative size");
  if (rows == 0 || T == 0) return MI_OK;
  if (!S) return fail(MI_ERR_NULL, "S is NULL");
  if (ld < T) return fail(MI_ERR_LD, "ld < T");
  if (rows > INT32_MAX) return fail(MI_ERR_SHAPE, "too many rows");
  if (dtype != MI_F32 && dtype != MI_BF16) return fail(MI_ERR_DTYPE, "dtype %d", dtype);
  int st = init_devices();
  if (st != MI_OK) return st;
  if (dtype == MI_BF16)
    hipLaunchKernelGGL(softmax_causal_kernel<true>, dim3((unsigned)rows), dim3(256), 0,
                       (hipStream_t)stream, S, T, ld);
  else
    hipLaunchKernelGGL(softmax_causal_kernel<false>, dim3((unsigned)rows), dim3(256), 0,
                       (hipStream_t)stream, S, T, ld);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MI_OK : fail(MI_ERR_HIP, "softmax: %s", hipGetErrorString(e));
}

int mi_softmax_bwd(void* stream, const void* P, void* dP, int64_t rows, int64_t T, int64_t ld,
                   float scale, int32_t dtype) {
  if (rows < 0 || T < 0) return fail(MI_ERR_SHAPE, "negative size");
  if (rows == 0 || T == 0) return MI_OK;
  if (!P || !dP) return fail(MI_ERR_NULL, "P or dP is NULL");
  if (ld < T) return fail(MI_ERR_LD, "ld < T");
  if (rows > INT32_MAX) return fail(MI_ERR_SHAPE, "too many rows");
  if (dtype != MI_F32 && dtype != MI_BF16) return fail(MI_ERR_DTYPE, "dtype %d", dtype);
  int st = init_devices();
  if (st != MI_OK) return st;
  if (dtype == MI_BF16)
    hipLaunchKernelGGL(softmax_bwd_kernel<true>, dim3((unsigned)rows), dim3(256), 0,
                       (hipStream_t)stream, P, dP, T, ld, scale);
  else
    hipLaunchKernelGGL(softmax_bwd_kernel<false>, dim3((unsigned)rows), dim3(256), 0,
                       (hipStream_t)stream, P, dP, T, ld, scale);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MI_OK : fail(MI_ERR_HIP, "softmax_bwd: %s", hipGetErrorString(e));
}

int mi_flash_attn_fwd(void* stream, const void* Q, const void* K, const void* V, void* O,
                      float* lse, int64_t batch, int64_t n_heads, int64_t n_kv, int64_t seq_len,
                      int64_t head_dim, int32_t causal, int32_t o_layout) {
  return mi_flash_attn_fwd_scaled(stream, Q, K, V, O, lse, batch, n_heads, n_kv, seq_len, head_dim,
                                  causal, o_layout, (float)(1.0 / std::sqrt((double)(head_dim > 0 ? head_dim : 1))));
}

int mi_flash_attn_fwd_scaled(void* stream, const void* Q, const void* K, const void* V, void* O,
                             float* lse, int64_t batch, int64_t n_heads, int64_t n_kv, int64_t seq_len,
                             int64_t head_dim, int32_t causal, int32_t o_layout, float scale) {
  if (batch < 0 || n_heads < 0 || n_kv < 0 || seq_len < 0)
    return fail(MI_ERR_SHAPE, "negative size");
  if (batch == 0 || n_heads == 0 || seq_len == 0) return MI_OK;
  if (!Q || !K || !V || !O) return fail(MI_ERR_NULL, "Q, K, V or O is NULL");
  if (n_kv <= 0 || n_heads % n_kv != 0)
    return fail(MI_ERR_SHAPE, "n_heads=%lld is not a multiple of n_kv=%lld", (long long)n_heads,
                (long long)n_kv);
  if (head_dim != 128 && head_dim != 64)
    return fail(MI_ERR_UNSUPPORTED, "flash attention supports head_dim 64 and 128 (got %lld)",
                (long long)head_dim);
  if (o_layout != MI_ATTN_O_BHTD && o_layout != MI_ATTN_O_BTHD)
    return fail(MI_ERR_SHAPE, "unknown output layout %d", o_layout);
  if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || ((uintptr_t)O & 7u) != 0 ||
      ((uintptr_t)lse & 3u) != 0)
    return fail(MI_ERR_UNSUPPORTED, "Q, K, V must be 16-byte aligned, O 8-byte, lse 4-byte");
  // every byte offset of one (batch, kv head) matrix and the block count fit 31 bits
  if (seq_len * head_dim * 2 >= ((int64_t)1 << 31) || batch * n_heads * seq_len > INT32_MAX)
    return fail(MI_ERR_SHAPE, "sequence too long");
  int st = init_devices();
  if (st != MI_OK) return st;
  FaParams p;
  p.Q = Q; p.K = K; p.V = V; p.O = O; p.lse = lse;
  p.B = (int)batch; p.nH = (int)n_heads; p.nKV = (int)n_kv; p.T = (int)seq_len;
  p.group = (int)(n_heads / n_kv);
  p.causal = causal != 0;
  p.o_bthd = o_layout == MI_ATTN_O_BTHD;
  p.q_blocks = flash_fwd_blocks(p.T);
  if (!(scale > 0.0f) || !std::isfinite(scale)) return fail(MI_ERR_SHAPE, "softmax scale must be positive");
  p.scale_log2 = (float)(1.4426950408889634 * (double)scale);
  if ((int64_t)p.B * p.nH * p.q_blocks > INT32_MAX) return fail(MI_ERR_SHAPE, "too many blocks");
  hipError_t e = launch_flash_fwd(p, (int)head_dim, (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : fail(MI_ERR_HIP, "flash attention launch: %s", hipGetErrorString(e));
}

// dS^T (bf16), then room for the fp32 dK / dV partials of the balanced dK/dV schedule.
static size_t flash_dst_bytes(int64_t batch, int64_t n_heads, int64_t seq_len) {
  // The dK/dV kernel stores dS^T in runs of 8 queries through 32-bit buffer offsets.
  if (batch <= 0 || n_heads <= 0 || seq_len <= 0 || seq_len % 8 || seq_len > 32767) return 0;
  return (size_t)batch * (size_t)n_heads * (size_t)seq_len * (size_t)seq_len * 2;
}

size_t mi_flash_attn_bwd_workspace_size(int64_t batch, int64_t n_heads, int64_t seq_len) {
  const size_t dst = flash_dst_bytes(batch, n_heads, seq_len);
  return dst ? dst + flash_bwd_partial_bytes(batch, n_heads, seq_len) : 0;
}

int mi_flash_attn_bwd(void* stream, const void* Q, const void* K, const void* V, const void* O,
                      const void* dO, const float* lse, void* dQ, void* dK, void* dV, float* delta,
                      int64_t batch, int64_t n_heads, int64_t n_kv, int64_t seq_len,
                      int64_t head_dim, int32_t causal, int32_t o_layout, void* workspace,
                      size_t workspace_bytes) {
  return mi_flash_attn_bwd_scaled(stream, Q, K, V, O, dO, lse, dQ, dK, dV, delta, batch, n_heads, n_kv,
                                  seq_len, head_dim, causal, o_layout, workspace, workspace_bytes,
                                  (float)(1.0 / std::sqrt((double)(head_dim > 0 ? head_dim : 1))));
}

int mi_flash_attn_bwd_scaled(void* stream, const void* Q, const void* K, const void* V, const void* O,
                             const void* dO, const float* lse, void* dQ, void* dK, void* dV, float* delta,
                             int64_t batch, int64_t n_heads, int64_t n_kv, int64_t seq_len,
                             int64_t head_dim, int32_t causal, int32_t o_layout, void* workspace,
                             size_t workspace_bytes, float scale) {
  if (batch < 0 || n_heads < 0 || n_kv < 0 || seq_len < 0)
    return fail(MI_ERR_SHAPE, "negative size");
  if (batch == 0 || n_heads == 0 || seq_len == 0) return MI_OK;
  if (!Q || !K || !V || !O || !dO || !lse || !dQ || !dK || !dV || !delta)
    return fail(MI_ERR_NULL, "an operand of the attention backward is NULL");
  if (n_kv <= 0 || n_heads % n_kv != 0)
    return fail(MI_ERR_SHAPE, "n_heads=%lld is not a multiple of n_kv=%lld", (long long)n_heads,
                (long long)n_kv);
  if (head_dim != 128 && head_dim != 64)
    return fail(MI_ERR_UNSUPPORTED, "flash attention supports head_dim 64 and 128 (got %lld)",
                (long long)head_dim);
  if (o_layout != MI_ATTN_O_BHTD && o_layout != MI_ATTN_O_BTHD)
    return fail(MI_ERR_SHAPE, "unknown output layout %d", o_layout);
  const void* a16[] = {Q, K, V, O, dO};
  for (const void* q : a16)
    if (!aligned16(q)) return fail(MI_ERR_UNSUPPORTED, "Q, K, V, O, dO must be 16-byte aligned");
  if (((uintptr_t)dQ & 7u) || ((uintptr_t)dK & 7u) || ((uintptr_t)dV & 7u) || ((uintptr_t)lse & 15u) ||
      ((uintptr_t)delta & 15u))
    return fail(MI_ERR_UNSUPPORTED, "dQ, dK, dV must be 8-byte aligned, lse and delta 16-byte");
  if (seq_len * head_dim * 2 * (o_layout == MI_ATTN_O_BTHD ? n_heads : 1) >= ((int64_t)1 << 31) ||
      batch * n_heads * seq_len > INT32_MAX)
    return fail(MI_ERR_SHAPE, "sequence too long");
  int st = init_devices();
  if (st != MI_OK) return st;
  FbParams p;
  p.Q = Q; p.K = K; p.V = V; p.O = O; p.dO = dO; p.lse = lse;
  p.dQ = dQ; p.dK = dK; p.dV = dV; p.delta = delta;
  p.B = (int)batch; p.nH = (int)n_heads; p.nKV = (int)n_kv; p.T = (int)seq_len;
  p.group = (int)(n_heads / n_kv);
  p.causal = causal != 0;
  p.o_bthd = o_layout == MI_ATTN_O_BTHD;
  p.q_blocks = flash_fwd_blocks(p.T);
  p.k_blocks = flash_bwd_key_blocks(p.T);
  if (!(scale > 0.0f) || !std::isfinite(scale)) return fail(MI_ERR_SHAPE, "softmax scale must be positive");
  p.scale = scale;
  p.scale_log2 = (float)(1.4426950408889634 * (double)scale);
  // With room for dS^T the dK/dV kernel writes it and dQ = scale * dS K is one batched
  // GEMM (5 MFMA products instead of 7); otherwise the dQ kernel recomputes S and dP.
  // Room beyond dS^T holds the partials of the balanced dK/dV schedule.
  const size_t need = flash_dst_bytes(batch, n_heads, seq_len);
  p.dsT = (workspace && need && workspace_bytes >= need && aligned16(workspace)) ? workspace : nullptr;
  p.part = p.dsT ? (float*)((char*)workspace + need) : nullptr;
  p.part_bytes = p.dsT ? workspace_bytes - need : 0;
  p.cus = current_cus();
  p.n_units = p.n_slots = p.n_split = 0;
  if (p.dsT && causal) {
    // Causal skipping in the dQ GEMM works on whole K tiles up to the end of a
    // 128-row output tile; the dK/dV kernel writes dS^T (zeros included) for every
    // key below that bound, and not beyond it, so taller tiles take the dQ kernel.
    const Plan pl = make_plan(MI_BF16, seq_len, head_dim, seq_len, batch * n_heads, MODE_PLAIN, false, 0,
                              current_cus(), true);
    if (shape_of(MI_BF16, pl.cfg).bm != 128) p.dsT = nullptr;
  }
  hipError_t e = launch_flash_bwd(p, (int)head_dim, (hipStream_t)stream);
  if (e != hipSuccess)
    return fail(MI_ERR_HIP, "flash attention backward launch: %s", hipGetErrorString(e));
  if (!p.dsT) return MI_OK;
  const int64_t T = seq_len, d = head_dim, g = n_heads / n_kv;
  mi_batch bt;
  std::memset(&bt, 0, sizeof(bt));
  bt.batch = batch * n_heads; bt.heads = n_heads;
  bt.a_outer = n_heads * T * T; bt.a_inner = T * T; bt.a_group = 1;   // dS^T [b][h][key][query]
  bt.b_outer = n_kv * T * d; bt.b_inner = T * d; bt.b_group = g;      // K of the head's KV head
  bt.c_outer = n_heads * T * d; bt.c_inner = T * d; bt.c_group = 1;   // dQ [b][h][query][d]
  bt.k_segments = 1;
  bt.causal = causal ? MI_CAUSAL_A_LOWER : MI_CAUSAL_NONE;            // dS[q][k] = 0 for k > q
  return mi_gemm_batched(stream, 1, 0, T, d, T, p.scale, p.dsT, T, K, d, MI_BF16, 0.0f, dQ, d, MI_BF16,
                         &bt, nullptr, nullptr, 0);
}

size_t mi_rmsnorm_bwd_workspace_size(int64_t rows, int64_t dims) {
  if (rows <= 0 || dims <= 0 || rows > INT32_MAX || dims > INT32_MAX) return 0;
  return (size_t)norm_bwd_grid((int)rows) * (size_t)dims * sizeof(float);
}

int mi_rmsnorm_fwd(void* stream, void* x, const void* residual, const void* weight, int32_t w_dtype,
                   void* y, float* rstd, int64_t rows, int64_t dims, int64_t ld, int32_t dtype,
                   float eps) {
  if (rows < 0 || dims < 0) return fail(MI_ERR_SHAPE, "negative size");
  if (rows == 0 || dims == 0) return MI_OK;
  if (rows > INT32_MAX || dims > INT32_MAX) return fail(MI_ERR_SHAPE, "size exceeds 2^31-1");
  if ((dtype != MI_F32 && dtype != MI_BF16) || (w_dtype != MI_F32 && w_dtype != MI_BF16))
    return fail(MI_ERR_DTYPE, "dtype %d / weight dtype %d", dtype, w_dtype);
  if (!x || !weight || (!y && !rstd)) return fail(MI_ERR_NULL, "x, weight, or both y and rstd are NULL");
  if (ld < dims) return fail(MI_ERR_LD, "ld=%lld < dims=%lld", (long long)ld, (long long)dims);
  const int64_t es = dtype == MI_BF16 ? 2 : 4, wes = w_dtype == MI_BF16 ? 2 : 4;
  const void* rows_arr[] = {x, y, residual};
  for (const void* q : rows_arr)
    if ((uintptr_t)q % es) return fail(MI_ERR_UNSUPPORTED, "row arrays must be aligned to their element size");
  if ((uintptr_t)weight % wes || ((uintptr_t)rstd & 3u))
    return fail(MI_ERR_UNSUPPORTED, "weight and rstd must be aligned to their element size");
  const int64_t extent = ((rows - 1) * ld + dims) * es;
  if (rows_overlap(y, x, extent) || rows_overlap(y, residual, extent) || rows_overlap(x, residual, extent))
    return fail(MI_ERR_UNSUPPORTED, "x, residual and y must each be the same array or disjoint");
  const int64_t ev = 16 / es;
  const bool vector_path = dims % ev == 0 && (ld * es) % 16 == 0 && aligned16(x) && (!y || aligned16(y)) &&
                           (!residual || aligned16(residual)) &&
                           (uintptr_t)weight % (w_dtype == MI_BF16 && ev == 4 ? 8 : 16) == 0 &&
                           dims / ev <= 64 * NORM_MAX_VEC_PER_LANE;
  int st = init_devices();
  if (st != MI_OK) return st;
  NormParams p{};
  p.x = x; p.r = residual; p.w = weight; p.y = y; p.rstd = rstd;
  p.ld = ld; p.rows = (int)rows; p.dims = (int)dims; p.eps = eps;
  hipError_t e = launch_norm_fwd(p, dtype == MI_BF16, w_dtype == MI_BF16, vector_path, (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : fail(MI_ERR_HIP, "rmsnorm_fwd launch: %s", hipGetErrorString(e));
}

int mi_rmsnorm_fold_weight(void* stream, const void* weight, int32_t w_dtype, const void* W, int64_t ldw,
                           int64_t K, int64_t N, int32_t dtype, void* W_out, int64_t ld_out) {
  if (K < 0 || N < 0) return fail(MI_ERR_SHAPE, "negative size");
  if (K == 0 || N == 0) return MI_OK;
  if ((dtype != MI_F32 && dtype != MI_BF16) || (w_dtype != MI_F32 && w_dtype != MI_BF16))
    return fail(MI_ERR_DTYPE, "dtype %d / weight dtype %d", dtype, w_dtype);
  if (!weight || !W || !W_out) return fail(MI_ERR_NULL, "weight, W or W_out is NULL");
  if (ldw < N || ld_out < N) return fail(MI_ERR_LD, "ldw=%lld / ld_out=%lld < N=%lld", (long long)ldw,
                                         (long long)ld_out, (long long)N);
  if (K > INT32_MAX || N > INT32_MAX) return fail(MI_ERR_SHAPE, "size exceeds 2^31-1");
  const int64_t es = dtype == MI_BF16 ? 2 : 4, wes = w_dtype == MI_BF16 ? 2 : 4;
  if ((uintptr_t)W % es || (uintptr_t)W_out % es || (uintptr_t)weight % wes)
    return fail(MI_ERR_UNSUPPORTED, "arrays must be aligned to their element size");
  const int64_t ext_in = ((K - 1) * ldw + N) * es, ext_out = ((K - 1) * ld_out + N) * es;
  if (W != W_out && rows_overlap(W_out, W, std::max(ext_in, ext_out)))
    return fail(MI_ERR_UNSUPPORTED, "W_out must be W itself or disjoint from it");
  if (W == W_out && ldw != ld_out) return fail(MI_ERR_LD, "in place needs ld_out == ldw");
  const int64_t ev = 16 / es;
  const bool vec = N % ev == 0 && ldw % ev == 0 && ld_out % ev == 0 && aligned16(W) && aligned16(W_out);
  int st = init_devices();
  if (st != MI_OK) return st;
  hipError_t e = launch_norm_fold_weight(weight, w_dtype == MI_BF16, W, ldw, K, N, dtype == MI_BF16, W_out,
                                         ld_out, vec, current_cus(), (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : fail(MI_ERR_HIP, "rmsnorm weight fold launch: %s", hipGetErrorString(e));
}

int mi_rmsnorm_bwd(void* stream, const void* dy, const void* x, const void* weight, int32_t w_dtype,
                   const void* residual_grad, void* dx, void* dw, int32_t dw_dtype, float dw_beta,
                   int64_t rows, int64_t dims, int64_t ld, int32_t dtype, float eps,
                   void* workspace, size_t workspace_bytes) {
  if (rows < 0 || dims < 0) return fail(MI_ERR_SHAPE, "negative size");
  if (rows == 0 || dims == 0) return MI_OK;
  if (rows > INT32_MAX || dims > INT32_MAX) return fail(MI_ERR_SHAPE, "size exceeds 2^31-1");
  if ((dtype != MI_F32 && dtype != MI_BF16) || (w_dtype != MI_F32 && w_dtype != MI_BF16) ||
      (dw && dw_dtype != MI_F32 && dw_dtype != MI_BF16))
    return fail(MI_ERR_DTYPE, "dtype %d / weight dtype %d / dw dtype %d", dtype, w_dtype, dw_dtype);
  if (!dy || !x || !weight || !dx) return fail(MI_ERR_NULL, "dy, x, weight or dx is NULL");
  if (ld < dims) return fail(MI_ERR_LD, "ld=%lld < dims=%lld", (long long)ld, (long long)dims);
  const size_t need = mi_rmsnorm_bwd_workspace_size(rows, dims);
  if (dw && (!workspace || workspace_bytes < need))
    return fail(MI_ERR_WORKSPACE, "dw needs %zu workspace bytes (got %zu)", need, workspace ? workspace_bytes : 0);
  const int64_t es = dtype == MI_BF16 ? 2 : 4, wes = w_dtype == MI_BF16 ? 2 : 4;
  const void* rows_arr[] = {dy, x, dx, residual_grad};
  for (const void* q : rows_arr)
    if ((uintptr_t)q % es) return fail(MI_ERR_UNSUPPORTED, "row arrays must be aligned to their element size");
  if ((uintptr_t)weight % wes || (dw && (uintptr_t)dw % (dw_dtype == MI_BF16 ? 2 : 4)) ||
      ((uintptr_t)workspace & 3u))
    return fail(MI_ERR_UNSUPPORTED, "weight, dw and workspace must be aligned to their element size");
  const int64_t extent = ((rows - 1) * ld + dims) * es;
  if (rows_overlap(dx, dy, extent) || rows_overlap(dx, x, extent) || rows_overlap(dx, residual_grad, extent))
    return fail(MI_ERR_UNSUPPORTED, "dx and each input must be the same array or disjoint");
  const int64_t ev = 16 / es;
  const bool vector_path = dims % ev == 0 && (ld * es) % 16 == 0 && aligned16(dy) && aligned16(x) &&
                           aligned16(dx) && (!residual_grad || aligned16(residual_grad)) &&
                           (uintptr_t)weight % (w_dtype == MI_BF16 && ev == 4 ? 8 : 16) == 0 &&
                           dims / ev <= 64 * NORM_MAX_VEC_PER_LANE;
  int st = init_devices();
  if (st != MI_OK) return st;
  NormParams p{};
  p.x = (void*)x; p.r = residual_grad; p.w = weight; p.dy = dy; p.dx = dx; p.dw = dw;
  p.ws = (float*)workspace;
  p.ld = ld; p.rows = (int)rows; p.dims = (int)dims; p.eps = eps; p.dw_beta = dw_beta;
  hipError_t e = launch_norm_bwd(p, dtype == MI_BF16, w_dtype == MI_BF16, dw_dtype == MI_BF16,
                                 vector_path, (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : fail(MI_ERR_HIP, "rmsnorm_bwd launch: %s", hipGetErrorString(e));
}

}  // extern "C"

namespace {

// Argument checks of one conversion (mi_convert_matrix, and each job of
// mi_convert_matrices; `what` names the job in messages).  On success fills p and the
// byte extents [s0, s1) of the source rows read and [d0, d1) of the destination
// rows written; an empty conversion returns MI_OK with p.rows or p.cols 0.
int check_convert(const void* src, int32_t src_dtype, int64_t src_ld, int64_t row0, int64_t rows,
                  int64_t cols, int32_t transpose, void* dst, int32_t dst_dtype, int64_t dst_ld,
                  const char* what, ConvParams& p, uintptr_t& s0, uintptr_t& s1, uintptr_t& d0,
                  uintptr_t& d1) {
  p = ConvParams{};
  s0 = s1 = d0 = d1 = 0;
  if (rows < 0 || cols < 0 || row0 < 0) return fail(MI_ERR_SHAPE, "%snegative size or row offset", what);
  if (rows == 0 || cols == 0) return MI_OK;
  if (src_dtype != MI_F32 && src_dtype != MI_BF16 && src_dtype != MI_F16)
    return fail(MI_ERR_DTYPE, "%ssource dtype %d", what, src_dtype);
  if (dst_dtype != MI_F32 && dst_dtype != MI_BF16)
    return fail(MI_ERR_DTYPE, "%sdestination dtype %d", what, dst_dtype);
  if (!src || !dst) return fail(MI_ERR_NULL, "%ssrc or dst is NULL", what);
  if (src_ld < cols)
    return fail(MI_ERR_LD, "%ssrc_ld=%lld < cols=%lld", what, (long long)src_ld, (long long)cols);
  if (dst_ld < (transpose ? rows : cols))
    return fail(MI_ERR_LD, "%sdst_ld=%lld < %lld", what, (long long)dst_ld,
                (long long)(transpose ? rows : cols));
  if (transpose && (rows + 63) / 64 > 65535) return fail(MI_ERR_SHAPE, "%stoo many rows to transpose", what);
  const int64_t ses = src_dtype == MI_F32 ? 4 : 2, des = dst_dtype == MI_F32 ? 4 : 2;
  if ((uintptr_t)src % ses || (uintptr_t)dst % des)
    return fail(MI_ERR_UNSUPPORTED, "%ssrc and dst must be aligned to their element size", what);
  s0 = (uintptr_t)src + (uintptr_t)(row0 * src_ld * ses);
  s1 = (uintptr_t)src + (uintptr_t)(((row0 + rows - 1) * src_ld + cols) * ses);
  const int64_t drows = transpose ? cols : rows, dcols = transpose ? rows : cols;
  d0 = (uintptr_t)dst;
  d1 = d0 + (uintptr_t)(((drows - 1) * dst_ld + dcols) * des);
  if (d0 < s1 && s0 < d1) return fail(MI_ERR_UNSUPPORTED, "%sdst overlaps the source rows", what);
  p.src = src; p.dst = dst; p.src_ld = src_ld; p.dst_ld = dst_ld;
  p.row0 = row0; p.rows = rows; p.cols = cols;
  p.src_dtype = src_dtype; p.dst_dtype = dst_dtype;
  return MI_OK;
}

}  // namespace

extern "C" {

int mi_convert_matrix(void* stream, const void* src, int32_t src_dtype, int64_t src_ld, int64_t row0,
                      int64_t rows, int64_t cols, int32_t transpose, void* dst, int32_t dst_dtype,
                      int64_t dst_ld) {
  ConvParams p;
  uintptr_t s0, s1, d0, d1;
  int st = check_convert(src, src_dtype, src_ld, row0, rows, cols, transpose, dst, dst_dtype, dst_ld,
                         "", p, s0, s1, d0, d1);
  if (st != MI_OK || p.rows == 0 || p.cols == 0) return st;
  st = init_devices();
  if (st != MI_OK) return st;
  hipError_t e = launch_convert(p, transpose != 0, current_cus(), (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : fail(MI_ERR_HIP, "convert launch: %s", hipGetErrorString(e));
}

int mi_convert_matrices(void* stream, const mi_convert_job* jobs, int64_t n) {
  if (n < 0) return fail(MI_ERR_SHAPE, "negative job count");
  if (n == 0) return MI_OK;
  if (!jobs) return fail(MI_ERR_NULL, "jobs is NULL");
  std::vector<ConvParams> ps((size_t)n);
  std::vector<int> tr((size_t)n);
  // byte extents: (begin, end, is_destination), swept in order of begin
  struct Extent { uintptr_t b, e; int dst; int64_t job; };
  std::vector<Extent> ext;
  ext.reserve(2 * (size_t)n);
  for (int64_t i = 0; i < n; ++i) {
    const mi_convert_job& j = jobs[i];
    char what[48];
    std::snprintf(what, sizeof what, "job %lld: ", (long long)i);
    if (j.reserved != 0)
      return fail(MI_ERR_SHAPE, "job %lld: reserved field is %d, must be 0", (long long)i, (int)j.reserved);
    uintptr_t s0, s1, d0, d1;
    const int st = check_convert(j.src, j.src_dtype, j.src_ld, j.row0, j.rows, j.cols, j.transpose, j.dst,
                                 j.dst_dtype, j.dst_ld, what, ps[(size_t)i], s0, s1, d0, d1);
    if (st != MI_OK) return st;
    tr[(size_t)i] = j.transpose != 0;
    if (ps[(size_t)i].rows == 0 || ps[(size_t)i].cols == 0) continue;
    ext.push_back({s0, s1, 0, i});
    ext.push_back({d0, d1, 1, i});
  }
  if (ext.empty()) return MI_OK;
  // A destination may not overlap any other extent; sources may share bytes.
  std::sort(ext.begin(), ext.end(), [](const Extent& x, const Extent& y) { return x.b < y.b; });
  uintptr_t end_any = 0, end_dst = 0;
  int64_t job_any = -1, job_dst = -1;
  for (const Extent& x : ext) {
    if (x.dst && x.b < end_any)
      return fail(MI_ERR_UNSUPPORTED, "job %lld: dst overlaps the source or destination of job %lld",
                  (long long)x.job, (long long)job_any);
    if (!x.dst && x.b < end_dst)
      return fail(MI_ERR_UNSUPPORTED, "job %lld: source rows overlap the destination of job %lld",
                  (long long)x.job, (long long)job_dst);
    if (x.e > end_any) end_any = x.e, job_any = x.job;
    if (x.dst && x.e > end_dst) end_dst = x.e, job_dst = x.job;
  }
  const int st = init_devices();
  if (st != MI_OK) return st;
  hipError_t e = launch_convert_batch(ps.data(), tr.data(), n, (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : fail(MI_ERR_HIP, "convert launch: %s", hipGetErrorString(e));
}

int mi_cross_entropy(void* stream, const void* logits, int32_t logits_dtype, int64_t ld_logits,
                     const uint32_t* targets, int64_t rows, int64_t vocab, float scale,
                     float* row_loss, float* loss_out, void* grad, int32_t grad_dtype,
                     int64_t ld_grad) {
  if (rows < 0 || vocab < 0) return fail(MI_ERR_SHAPE, "negative size");
  if (rows == 0 || vocab == 0) return MI_OK;
  if (rows > INT32_MAX || vocab > INT32_MAX) return fail(MI_ERR_SHAPE, "size exceeds 2^31-1");
  if (logits_dtype != MI_F32 && logits_dtype != MI_BF16)
    return fail(MI_ERR_DTYPE, "logits dtype %d", logits_dtype);
  if (grad && grad_dtype != MI_F32 && grad_dtype != MI_BF16)
    return fail(MI_ERR_DTYPE, "grad dtype %d", grad_dtype);
  if (!logits || !targets || !row_loss) return fail(MI_ERR_NULL, "logits, targets or row_loss is NULL");
  if (ld_logits < vocab) return fail(MI_ERR_LD, "ld_logits=%lld < vocab=%lld", (long long)ld_logits,
                                     (long long)vocab);
  if (grad && ld_grad < vocab)
    return fail(MI_ERR_LD, "ld_grad=%lld < vocab=%lld", (long long)ld_grad, (long long)vocab);
  const int64_t in_es = logits_dtype == MI_BF16 ? 2 : 4, out_es = grad_dtype == MI_BF16 ? 2 : 4;
  if (((uintptr_t)logits % in_es) || ((uintptr_t)targets & 3u) || ((uintptr_t)row_loss & 3u) ||
      ((uintptr_t)loss_out & 3u) || (grad && ((uintptr_t)grad % out_es)))
    return fail(MI_ERR_UNSUPPORTED, "pointers must be aligned to their element size");
  if (grad) {  // in place only as an exact alias of the logits
    const uintptr_t l0 = (uintptr_t)logits, l1 = l0 + (uintptr_t)(((rows - 1) * ld_logits + vocab) * in_es);
    const uintptr_t g0 = (uintptr_t)grad, g1 = g0 + (uintptr_t)(((rows - 1) * ld_grad + vocab) * out_es);
    if (g0 < l1 && l0 < g1 &&
        !(g0 == l0 && grad_dtype == logits_dtype && ld_grad == ld_logits))
      return fail(MI_ERR_UNSUPPORTED, "grad overlaps logits without being the same array");
  }
  const int64_t ev = 16 / in_es;
  const int64_t out_vec = ev * out_es;  // bytes one vector's gradient occupies
  const int64_t out_align = out_vec < 16 ? out_vec : 16;
  const bool vector_path = vocab % ev == 0 && aligned16(logits) && (ld_logits * in_es) % 16 == 0 &&
                           vocab / ev <= (int64_t)XENT_THREADS * XENT_MAX_VEC_PER_THREAD &&
                           (!grad || ((uintptr_t)grad % out_align == 0 && (ld_grad * out_es) % out_align == 0));
  int st = init_devices();
  if (st != MI_OK) return st;
  XentParams p;
  p.logits = logits; p.targets = targets; p.row_loss = row_loss; p.grad = grad;
  p.ld = ld_logits; p.ldg = grad ? ld_grad : 0;
  p.rows = (int)rows; p.vocab = (int)vocab;
  p.scale = scale;
  hipError_t e = launch_xent(p, logits_dtype == MI_BF16, grad && grad_dtype == MI_BF16, vector_path,
                             (hipStream_t)stream);
  if (e == hipSuccess && loss_out) e = launch_xent_mean(row_loss, (int)rows, scale, loss_out, (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : fail(MI_ERR_HIP, "cross_entropy launch: %s", hipGetErrorString(e));
}

}  // extern "C"

namespace {

// Workspace carve of mi_lm_head_xent: the bf16 logits chunk [rows][lm_chunk_ld], three fp32
// row arrays (running max, running sum then scale / sum, target logit), and an fp32
// [rows][hidden] accumulator of dX when dX is bf16; each part 256-byte aligned, plus 256
// bytes for aligning the base.  What is left over is split-K workspace for the GEMMs.
// The chunk's row pitch is a whole number of 16-byte vectors, plus 256 bytes when it
// would be a multiple of 2 KB: with a 16 KB pitch (chunks of 8192) every row of a C
// tile starts at the same offset of the 4 KB period the memory channels interleave
// over, and the chunk GEMMs ran 1080 / 1251 / 1319 TFLOP/s (logits, dX, dW) against
// 1289 / 1320 / 1345 with the pitch padded (configuration 5, one box).
int64_t lm_chunk_ld(int64_t chunk) {
  const int64_t ld = (chunk + 7) / 8 * 8;
  return ld % 1024 == 0 ? ld + 128 : ld;
}
size_t align256(size_t b) { return (b + 255) / 256 * 256; }
size_t lm_fixed_bytes(int64_t rows, int64_t hidden, int64_t chunk, bool dx_acc) {
  return 256 + align256((size_t)rows * (size_t)lm_chunk_ld(chunk) * 2) + 3 * align256((size_t)rows * 4) +
         (dx_acc ? align256((size_t)rows * (size_t)hidden * 4) : 0);
}

int lm_gemm(hipStream_t st, int tA, int tB, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
            const void* B, int64_t ldb, float beta, void* C, int64_t ldc, int32_t dtype_c, void* ws,
            size_t ws_bytes) {
  Problem P;
  P.transA = tA; P.transB = tB;
  P.M = M; P.N = N; P.K = K;
  P.alpha = 1.0f; P.beta = beta;
  P.A = A; P.B = B; P.lda = lda; P.ldb = ldb;
  P.dtype_in = MI_BF16;
  P.C = C; P.ldc = ldc; P.dtype_c = dtype_c;
  P.bt = single_batch();
  std::memset(&P.ep, 0, sizeof(P.ep));
  P.ws = ws;
  P.ws_bytes = ws_bytes;
  return run(P, st);
}

}  // namespace

extern "C" {

size_t mi_lm_head_xent_workspace_size(int64_t rows, int64_t hidden, int64_t vocab, int64_t chunk,
                                      int32_t dx_dtype) {
  if (rows <= 0 || hidden <= 0 || vocab <= 0) return 0;
  if (chunk <= 0 || chunk > vocab) chunk = vocab;
  return lm_fixed_bytes(rows, hidden, chunk, dx_dtype == MI_BF16);
}

int mi_lm_head_xent(void* stream, const void* X, int64_t ldx, const void* W, int32_t w_layout, int64_t ldw,
                    const uint32_t* targets, int64_t rows, int64_t hidden, int64_t vocab, float scale,
                    float* row_loss, float* loss_out, void* dX, int32_t dx_dtype, int64_t lddx, void* dW,
                    int32_t dw_dtype, int64_t lddw, float dw_beta, int64_t chunk, void* workspace,
                    size_t workspace_bytes) {
  if (rows < 0 || hidden < 0 || vocab < 0) return fail(MI_ERR_SHAPE, "negative size");
  if (rows == 0 || vocab == 0) return MI_OK;
  if (hidden == 0) return fail(MI_ERR_SHAPE, "hidden = 0");
  if (rows > INT32_MAX || hidden > INT32_MAX || vocab > INT32_MAX)
    return fail(MI_ERR_SHAPE, "size exceeds 2^31-1");
  if (w_layout != 0 && w_layout != 1) return fail(MI_ERR_UNSUPPORTED, "w_layout %d (0 or 1)", w_layout);
  if (!X || !W || !targets || !row_loss) return fail(MI_ERR_NULL, "X, W, targets or row_loss is NULL");
  if (ldx < hidden) return fail(MI_ERR_LD, "ldx=%lld < hidden=%lld", (long long)ldx, (long long)hidden);
  const int64_t w_row = w_layout == 0 ? vocab : hidden;
  if (ldw < w_row) return fail(MI_ERR_LD, "ldw=%lld < %lld", (long long)ldw, (long long)w_row);
  if (dX) {
    if (dx_dtype != MI_F32 && dx_dtype != MI_BF16) return fail(MI_ERR_DTYPE, "dX dtype %d", dx_dtype);
    if (lddx < hidden) return fail(MI_ERR_LD, "lddx=%lld < hidden=%lld", (long long)lddx, (long long)hidden);
  }
  if (dW) {
    if (dw_dtype != MI_F32 && dw_dtype != MI_BF16) return fail(MI_ERR_DTYPE, "dW dtype %d", dw_dtype);
    if (lddw < w_row) return fail(MI_ERR_LD, "lddw=%lld < %lld", (long long)lddw, (long long)w_row);
  }
  if (((uintptr_t)X & 1u) || ((uintptr_t)W & 1u) || ((uintptr_t)targets & 3u) || ((uintptr_t)row_loss & 3u) ||
      ((uintptr_t)loss_out & 3u))
    return fail(MI_ERR_UNSUPPORTED, "pointers must be aligned to their element size");
  if (chunk <= 0 || chunk > vocab) chunk = vocab;
  const bool dx_acc = dX && dx_dtype == MI_BF16;
  const size_t need = lm_fixed_bytes(rows, hidden, chunk, dx_acc);
  if (!workspace || workspace_bytes < need)
    return fail(MI_ERR_WORKSPACE, "workspace of %zu bytes < %zu (mi_lm_head_xent_workspace_size)",
                workspace_bytes, need);
  const int st0 = init_devices();
  if (st0 != MI_OK) return st0;
  hipStream_t st = (hipStream_t)stream;
  // carve the workspace
  char* base = (char*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  const int64_t ldl = lm_chunk_ld(chunk);
  uint16_t* L = (uint16_t*)base;
  base += align256((size_t)rows * (size_t)ldl * 2);
  float* run_m = (float*)base;
  base += align256((size_t)rows * 4);
  float* run_s = (float*)base;
  base += align256((size_t)rows * 4);
  float* xy = (float*)base;
  base += align256((size_t)rows * 4);
  float* acc = nullptr;
  if (dx_acc) {
    acc = (float*)base;
    base += align256((size_t)rows * (size_t)hidden * 4);
  }
  void* gws = base;
  const size_t gws_bytes = workspace_bytes - (size_t)(base - (char*)workspace);
  const uint16_t* w16 = (const uint16_t*)W;
  const int64_t nchunks = (vocab + chunk - 1) / chunk;
  // logits of chunk c: L[rows][n] = X Wc, Wc = W[:, c0:c0+n] (layout 0) or W[c0:c0+n, :]^T (layout 1)
  auto logits = [&](int64_t c0, int64_t n) {
    return w_layout == 0 ? lm_gemm(st, 0, 0, rows, n, hidden, X, ldx, w16 + c0, ldw, 0.0f, L, ldl, MI_BF16, gws,
                                   gws_bytes)
                         : lm_gemm(st, 0, 1, rows, n, hidden, X, ldx, w16 + c0 * ldw, ldw, 0.0f, L, ldl, MI_BF16,
                                   gws, gws_bytes);
  };
  auto herr = [](hipError_t e) {
    return e == hipSuccess ? MI_OK : fail(MI_ERR_HIP, "lm_head_xent launch: %s", hipGetErrorString(e));
  };
  // pass 1: running (max, sum) over the chunks in order, then the row losses
  for (int64_t c = 0; c < nchunks; ++c) {
    const int64_t c0 = c * chunk, n = std::min(chunk, vocab - c0);
    int r = logits(c0, n);
    if (r != MI_OK) return r;
    r = herr(launch_xent_chunk_stats(L, ldl, (int)rows, (int)n, (int)c0, targets, run_m, run_s, xy, c == 0, st));
    if (r != MI_OK) return r;
  }
  int r = herr(launch_xent_chunk_finish((int)rows, (int)vocab, targets, run_m, run_s, xy, scale, row_loss, st));
  if (r == MI_OK && loss_out) r = herr(launch_xent_mean(row_loss, (int)rows, scale, loss_out, st));
  if (r != MI_OK || (!dX && !dW)) return r;
  // pass 2, last chunk first: its logits are still in L; every other chunk is recomputed
  void* dx_c = dx_acc ? (void*)acc : dX;
  const int64_t dx_ld = dx_acc ? hidden : lddx;
  const int32_t dx_t = dx_acc ? MI_F32 : dx_dtype;
  const int64_t esw = dw_dtype == MI_BF16 ? 2 : 4;
  for (int64_t c = nchunks - 1; c >= 0; --c) {
    const int64_t c0 = c * chunk, n = std::min(chunk, vocab - c0);
    if (c != nchunks - 1 && (r = logits(c0, n)) != MI_OK) return r;
    r = herr(launch_xent_chunk_grad(L, ldl, (int)rows, (int)n, (int)c0, targets, run_m, run_s, scale, st));
    if (r != MI_OK) return r;
    const float bx = c == nchunks - 1 ? 0.0f : 1.0f;
    if (dX) {  // dX (+)= dL_c Wc^T
      r = w_layout == 0 ? lm_gemm(st, 0, 1, rows, hidden, n, L, ldl, w16 + c0, ldw, bx, dx_c, dx_ld, dx_t, gws,
                                  gws_bytes)
                        : lm_gemm(st, 0, 0, rows, hidden, n, L, ldl, w16 + c0 * ldw, ldw, bx, dx_c, dx_ld, dx_t,
                                  gws, gws_bytes);
      if (r != MI_OK) return r;
    }
    if (dW) {  // dW's chunk = dw_beta dW's chunk + X^T dL_c (layout 0) or dL_c^T X (layout 1)
      r = w_layout == 0 ? lm_gemm(st, 1, 0, hidden, n, rows, X, ldx, L, ldl, dw_beta,
                                  (char*)dW + c0 * esw, lddw, dw_dtype, gws, gws_bytes)
                        : lm_gemm(st, 1, 0, n, hidden, rows, L, ldl, X, ldx, dw_beta,
                                  (char*)dW + c0 * lddw * esw, lddw, dw_dtype, gws, gws_bytes);
      if (r != MI_OK) return r;
    }
  }
  if (dx_acc) {
    ConvParams cp{};
    cp.src = acc; cp.dst = dX; cp.src_ld = hidden; cp.dst_ld = lddx;
    cp.row0 = 0; cp.rows = rows; cp.cols = hidden;
    cp.src_dtype = MI_F32; cp.dst_dtype = MI_BF16;
    r = herr(launch_convert(cp, false, current_cus(), st));
  }
  return r;
}

int mi_gemm_describe(int transA, int transB, int64_t M, int64_t N, int64_t K, int32_t dtype_in,
                     int64_t batch, int32_t epi_mode, size_t workspace_bytes, char* buf,
                     size_t buf_len) {
  if (!buf || buf_len == 0) return fail(MI_ERR_NULL, "buf is NULL");
  if (M <= 0 || N <= 0 || K < 0 || batch <= 0) return fail(MI_ERR_SHAPE, "bad shape");
  if (dtype_in != MI_F32 && dtype_in != MI_BF16) return fail(MI_ERR_DTYPE, "dtype %d", dtype_in);
  int cus = 256;
  if (init_devices() == MI_OK) cus = current_cus();
  const int mode = epi_mode == 1 ? MODE_DUAL : (epi_mode == 2 ? MODE_PROLOGUE : MODE_PLAIN);
  const int64_t ws = (int64_t)(workspace_bytes / sizeof(float));
  // packed operands (leading dimension = contiguous extent), 16-byte-aligned bases: the
  // 16-byte loaders need the contiguous extents in whole 16-byte chunks, as run() checks
  const int64_t ch = dtype_in == MI_BF16 ? 8 : 4;
  const int64_t a_contig = transA ? M : K, b_contig = transB ? K : N;
  const bool fast = K == 0 || (a_contig % ch == 0 && b_contig % ch == 0);
  const Plan pl = make_plan(dtype_in, M, N, K, batch, mode, ws > 0, ws, cus, fast);
  describe_plan(buf, buf_len, dtype_in, fast, pl, transA, transB, batch);
  return MI_OK;
}

int mi_profiler_enable(int on) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  const int was = g_prof_on ? 1 : 0;
  g_prof_on = on != 0;
  return was;
}

int mi_profiler_begin_step(void) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  int st = MI_OK;
  for (ProfEntry& en : g_prof) {
    if (prof_resolve(en) != MI_OK) st = MI_ERR_HIP;
    g_prof_free[en.dev].push_back(en.e0);
    g_prof_free[en.dev].push_back(en.e1);
  }
  g_prof.clear();
  return st;
}

int64_t mi_profiler_count(void) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  return (int64_t)g_prof.size();
}

int mi_profiler_record(int64_t i, mi_gemm_record* out) {
  if (!out) return fail(MI_ERR_NULL, "out is NULL");
  std::lock_guard<std::mutex> lk(g_prof_mu);
  if (i < 0 || i >= (int64_t)g_prof.size())
    return fail(MI_ERR_SHAPE, "record %lld of %zu", (long long)i, g_prof.size());
  const int st = prof_resolve(g_prof[(size_t)i]);
  if (st != MI_OK) return st;
  *out = g_prof[(size_t)i].rec;
  return MI_OK;
}

int mi_profiler_totals(double* gpu_ms, int64_t* calls) {
  if (!gpu_ms || !calls) return fail(MI_ERR_NULL, "gpu_ms or calls is NULL");
  std::lock_guard<std::mutex> lk(g_prof_mu);
  int st = MI_OK;
  for (ProfEntry& en : g_prof)
    if (prof_resolve(en) != MI_OK) st = MI_ERR_HIP;
  *gpu_ms = g_prof_total_ms;
  *calls = g_prof_calls;
  return st;
}

int mi_profiler_reset(void) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  int st = MI_OK;
  for (ProfEntry& en : g_prof)  // records keep their times; the totals restart from zero
    if (prof_resolve(en) != MI_OK) st = MI_ERR_HIP;
  g_prof_total_ms = 0.0;
  g_prof_calls = 0;
  return st;
}

int mi_stream_sync(void* stream) {
  hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  return e == hipSuccess ? MI_OK : fail(MI_ERR_HIP, "sync: %s", hipGetErrorString(e));
}

}  // extern "C"
