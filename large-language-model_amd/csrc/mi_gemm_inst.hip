// mi_gemm_inst.hip -- instantiates the GEMM kernels of one (dtype, transA,
// transB) combination.  Compiled once per combination with
//   -DMI_DT_BF16=0|1 -DMI_TA=0|1 -DMI_TB=0|1
#include "mi_gemm_dlds.hpp"
#include "mi_gemm_kernels.hpp"

#if !defined(MI_DT_BF16) || !defined(MI_TA) || !defined(MI_TB)
#error "define MI_DT_BF16, MI_TA and MI_TB"
#endif

namespace mig {

#if MI_DT_BF16
typedef __bf16 elem_t;
#define MI_DTN bf16
#else
typedef float elem_t;
#define MI_DTN f32
#endif
// ktail: the K extent of a segment is not a multiple of 64 (bf16 direct-to-LDS
// kernels then mask K-contiguous chunks past the end); fast_epi: the problem
// qualifies for the direct epilogue.  Both are ignored for fp32.

#ifndef MI_DLDS_BK
#define MI_DLDS_BK 64
#endif
#ifndef MI_DLDS_STAGES
#define MI_DLDS_STAGES 2
#endif
// 128x128: a K-contiguous A (NN, NT) runs the two-stage early-read ring at
// K tile 64; with A row-contiguous (TN, TT) the four-stage K-32 ring measured
// faster (2048x2048x8192 TN: 866 vs 672 TFLOP/s; 8192x3072x2048 NN: 991 vs 861).
#ifndef MI_S_BK
#define MI_S_BK(ak) ((ak) ? 64 : 32)
#endif
#ifndef MI_S_STAGES
#define MI_S_STAGES(ak) ((ak) ? 2 : 4)
#endif
// 128x128 with wave-level split-K (one workgroup of 8 waves per CU): K tile and
// ring depth.
#ifndef MI_W_STAGES
#define MI_W_STAGES 4
#endif
// 128x192 with wave-level split-K: ring depth (40 KB per stage at K tile 64).
#ifndef MI_V_STAGES
#define MI_V_STAGES 3
#endif
// 256x192 (8 waves of 64x96): K tile and ring depth by operand layout (ak: A is
// K-contiguous, bk: B is K-contiguous).
#ifndef MI_M_BK
#define MI_M_BK(ak, bk) MI_DLDS_BK
#endif
#ifndef MI_M_STAGES
#define MI_M_STAGES(ak, bk) MI_DLDS_STAGES
#endif
// 256x256 (8 waves of 128x64): K tile and ring depth by operand layout.
#ifndef MI_L_BK
#define MI_L_BK(ak, bk) MI_DLDS_BK
#endif
#ifndef MI_L_STAGES
#define MI_L_STAGES(ak, bk) MI_DLDS_STAGES
#endif

#define MI_CAT5(a, b, c, d, e) a##b##c##d##e
#define MI_PICK_NAME(dt, ta, tb) MI_CAT5(pick_, dt, _, ta, tb)

#if MI_DT_BF16
// bf16 direct-to-LDS kernels of one variant (K tile and LDS ring depth:
// MI_DLDS_BK / MI_DLDS_STAGES for 256x256, MI_S_BK / MI_S_STAGES of the A layout for 128x128,
// 32 / 4 for the dual-B 256x128).  256x256 runs 8 waves (2 x 4, wave tiles 128x64): two
// waves per SIMD, so one wave's MFMAs issue while the other waits on LDS or DMA issue
// (8192x2048x5632 NT: 147 vs 161 us with 4 waves of 128x128; 8192x5632x2048 NN 157 vs
// 166; 2048x5632x8192 TN 170 vs 180; bit-identical results).
template <bool AK, bool BK, int V>
KernelFn dlds_kernel(int cfg) {
  if constexpr ((V & DLDS_ROWSCALE) != 0) {
    // the row-scale epilogue (a folded RMSNorm) exists where the norm's GEMMs run: a
    // K-contiguous A on the 256x256, 256x192 and 128x128 tiles
    if constexpr (AK) {
      switch (cfg) {
        case CFG_L:
          return gemm_dlds_kernel<256, 256, MI_L_BK(AK, BK), MI_L_STAGES(AK, BK), AK, BK, MODE_PLAIN, V, 2, 4, 1>;
        case CFG_M:
          return gemm_dlds_kernel<256, 192, MI_M_BK(AK, BK), MI_M_STAGES(AK, BK), AK, BK, MODE_PLAIN, V, 4, 2, 1>;
        case CFG_S: return gemm_dlds_kernel<128, 128, MI_S_BK(AK), MI_S_STAGES(AK), AK, BK, MODE_PLAIN, V>;
        default: return nullptr;
      }
    }
    return nullptr;
  }
  switch (cfg) {
    case CFG_L:
      return gemm_dlds_kernel<256, 256, MI_L_BK(AK, BK), MI_L_STAGES(AK, BK), AK, BK, MODE_PLAIN, V, 2, 4, 1>;
    case CFG_S: return gemm_dlds_kernel<128, 128, MI_S_BK(AK), MI_S_STAGES(AK), AK, BK, MODE_PLAIN, V>;
    case CFG_DUAL: return gemm_dlds_kernel<256, 128, 32, 4, AK, BK, MODE_DUAL, V>;
    case CFG_W:
      return gemm_dlds_kernel<128, 128, MI_W_BK, MI_W_STAGES, AK, BK, MODE_PLAIN, V, 2, 2, 2>;
    case CFG_M:
      return gemm_dlds_kernel<256, 192, MI_M_BK(AK, BK), MI_M_STAGES(AK, BK), AK, BK, MODE_PLAIN, V, 4, 2, 1>;
    case CFG_V:
      return gemm_dlds_kernel<128, 192, MI_W_BK, MI_V_STAGES, AK, BK, MODE_PLAIN, V, 2, 2, 2>;
    default: return nullptr;
  }
}
#endif

#if !MI_DT_BF16
// fp32 direct-to-LDS kernels: K tile 32 (128-byte rows, the bytes of a bf16 K tile
// of 64), four 32x32x2 MFMAs per fragment pair and substep; 64x128 (four waves of
// 32x64) and 64x64 (four waves of 32x32).  The 64x128 tile replaced the register-
// staged kernel of that tile (configuration 2's set 89-91 -> 104-107 TFLOP/s, same
// box, two runs each).
template <bool AK, bool BK, int V>
KernelFn dlds32_kernel(int cfg) {
  switch (cfg) {
    case CFG_V: return gemm_dlds_kernel<64, 128, 32, 2, AK, BK, MODE_PLAIN, V, 2, 2, 1, 4>;
    case CFG_M: return gemm_dlds_kernel<64, 64, 32, 2, AK, BK, MODE_PLAIN, V, 2, 2, 1, 4>;
    default: return nullptr;
  }
}
#endif

KernelFn MI_PICK_NAME(MI_DTN, MI_TA, MI_TB)(int cfg, bool fast, bool ktail, int fast_epi) {
  constexpr bool AK = (MI_TA == 0);  // A is K-contiguous when not transposed
  constexpr bool BK = (MI_TB == 1);  // B is K-contiguous when transposed
#if MI_DT_BF16
  constexpr int LM = 256, LN = 256, SM = 128, SN = 128, DM = 256, DN = 128, PM = 256, PN = 256;
#else
  constexpr int LM = 128, LN = 128, SM = 128, SN = 128, DM = 128, DN = 64, PM = 128, PN = 128;
#endif
  if (fast) {
#if MI_DT_BF16
    if (cfg != CFG_PRO) {
      // K-tail variants exist only where an operand is K-contiguous; a K tail
      // takes the general epilogue.
      if constexpr (AK || BK) {
        if (ktail) return dlds_kernel<AK, BK, DLDS_KTAIL>(cfg);
      }
      if (fast_epi == 2) return dlds_kernel<AK, BK, DLDS_FAST_EPI | DLDS_ROWSCALE>(cfg);
      return fast_epi ? dlds_kernel<AK, BK, DLDS_FAST_EPI>(cfg) : dlds_kernel<AK, BK, 0>(cfg);
    }
    switch (cfg) {
      case CFG_PRO:
        if constexpr (AK) return gemm_kernel<elem_t, PM, PN, 2, 2, AK, BK, MODE_PROLOGUE, true>;
        return nullptr;
    }
#endif
#if !MI_DT_BF16
    if (cfg == CFG_V || cfg == CFG_M) {
      if constexpr (AK || BK) {
        if (ktail) return dlds32_kernel<AK, BK, DLDS_KTAIL>(cfg);
      }
      return fast_epi ? dlds32_kernel<AK, BK, DLDS_FAST_EPI>(cfg) : dlds32_kernel<AK, BK, 0>(cfg);
    }
#endif
    switch (cfg) {
      case CFG_L: return gemm_kernel<elem_t, LM, LN, 2, 2, AK, BK, MODE_PLAIN, true>;
      case CFG_S: return gemm_kernel<elem_t, SM, SN, 2, 2, AK, BK, MODE_PLAIN, true>;
      case CFG_DUAL: return gemm_kernel<elem_t, DM, DN, 2, 2, AK, BK, MODE_DUAL, true>;
      case CFG_PRO:
        if constexpr (AK) return gemm_kernel<elem_t, PM, PN, 2, 2, AK, BK, MODE_PROLOGUE, true>;
        return nullptr;
    }
  } else {
    switch (cfg) {
      case CFG_S: return gemm_kernel<elem_t, SM, SN, 2, 2, AK, BK, MODE_PLAIN, false>;
      case CFG_DUAL: return gemm_kernel<elem_t, DM, DN, 2, 2, AK, BK, MODE_DUAL, false>;
      case CFG_PRO:
        if constexpr (AK) return gemm_kernel<elem_t, PM, PN, 2, 2, AK, BK, MODE_PROLOGUE, false>;
        return nullptr;
      default: return nullptr;
    }
  }
  return nullptr;
}

}  // namespace mig
