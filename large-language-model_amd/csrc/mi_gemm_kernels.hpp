// mi_gemm_kernels.hpp -- kernel table shared by the host dispatch (mi_gemm.hip)
// and the per-layout instantiation units (mi_gemm_inst.hip, compiled once per
// input dtype x operand layout so the instantiations build in parallel).
#pragma once
#include "mi_gemm_device.hpp"

namespace mig {

typedef void (*KernelFn)(Params);

// Tile configurations.  Output tile (BM x BN) per configuration and dtype:
//   bf16: L 256x256 (8 waves of 128x64, two per SIMD), S 128x128 (4 waves of 64x64),
//         DUAL 256x128 (+ second B), PRO 256x256 with the SiLU-gate A prologue,
//         W 128x128 with wave-level split-K (8 waves: two groups of 4 waves of
//         64x64, each over half of every K tile, summed through LDS),
//         M 256x192 (8 waves of 64x96), V 128x192 with wave-level split-K (two
//         groups of 4 waves of 64x96).
//   fp32: V 64x128 and M 64x64 direct-to-LDS (four waves); register-staged
//         L = S = W 128x128, DUAL 128x64, PRO 128x128.
enum Cfg { CFG_L = 0, CFG_S = 1, CFG_DUAL = 2, CFG_PRO = 3, CFG_W = 4, CFG_M = 5, CFG_V = 6, NCFG = 7 };

struct CfgShape {
  int bm, bn;
  int threads = 256;  // workgroup size of the configuration's kernels
};

// K tile of the bf16 W configuration (its K-tail variant is needed when K is
// not a multiple of it).
#ifndef MI_W_BK
#define MI_W_BK 64
#endif

inline CfgShape cfg_shape(bool bf16, int cfg) {
  if (bf16)
    return cfg == CFG_L ? CfgShape{256, 256, 512}
         : cfg == CFG_S ? CfgShape{128, 128}
         : cfg == CFG_W ? CfgShape{128, 128, 512}
         : cfg == CFG_M ? CfgShape{256, 192, 512}
         : cfg == CFG_V ? CfgShape{128, 192, 512}
         : cfg == CFG_DUAL ? CfgShape{256, 128}
                           : CfgShape{256, 256};
  // fp32: V and M name the direct-to-LDS 64x128 and 64x64 tiles (four waves), the
  // others the register-staged kernel (four waves)
  return cfg == CFG_DUAL ? CfgShape{128, 64}
       : cfg == CFG_V    ? CfgShape{64, 128}
       : cfg == CFG_M    ? CfgShape{64, 64}
                         : CfgShape{128, 128};
}

// One function per (dtype, transA, transB): returns the kernel for `cfg` with
// the fast (buffer-load) or the element-granular loader, or nullptr when the
// combination does not exist (prologue with transA = 1).  The element-granular
// variant of the plain configurations exists only for CFG_S.  ktail: the K
// extent is not a multiple of 64; fast_epi (1, or 2 with the row scale): every tile is full and the
// epilogue is alpha (SiLU gate), beta*C and the output conversion only, with
// no split-K.
#define MI_DECL_PICK(dt, ta, tb) \
  KernelFn pick_##dt##_##ta##tb(int cfg, bool fast, bool ktail, int fast_epi);
MI_DECL_PICK(bf16, 0, 0)
MI_DECL_PICK(bf16, 0, 1)
MI_DECL_PICK(bf16, 1, 0)
MI_DECL_PICK(bf16, 1, 1)
MI_DECL_PICK(f32, 0, 0)
MI_DECL_PICK(f32, 0, 1)
MI_DECL_PICK(f32, 1, 0)
MI_DECL_PICK(f32, 1, 1)
#undef MI_DECL_PICK

}  // namespace mig
