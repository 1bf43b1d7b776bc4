// mi_gemm_inst.hip -- instantiates the GEMM kernels of one (dtype, transA,
// transB) combination.  Compiled once per combination with
//   -DMI_DT_BF16=0|1 -DMI_TA=0|1 -DMI_TB=0|1
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

#define MI_CAT5(a, b, c, d, e) a##b##c##d##e
#define MI_PICK_NAME(dt, ta, tb) MI_CAT5(pick_, dt, _, ta, tb)

KernelFn MI_PICK_NAME(MI_DTN, MI_TA, MI_TB)(int cfg) {
  constexpr bool AK = (MI_TA == 0);  // A is K-contiguous when not transposed
  constexpr bool BK = (MI_TB == 1);  // B is K-contiguous when transposed
#if MI_DT_BF16
  switch (cfg) {
    case CFG_L: return gemm_kernel<elem_t, 256, 256, 2, 2, AK, BK, MODE_PLAIN>;
    case CFG_S: return gemm_kernel<elem_t, 128, 128, 2, 2, AK, BK, MODE_PLAIN>;
    case CFG_DUAL: return gemm_kernel<elem_t, 256, 128, 2, 2, AK, BK, MODE_DUAL>;
    case CFG_PRO:
#if MI_TA == 0
      return gemm_kernel<elem_t, 256, 256, 2, 2, AK, BK, MODE_PROLOGUE>;
#else
      return nullptr;
#endif
  }
#else
  switch (cfg) {
    case CFG_L:
    case CFG_S: return gemm_kernel<elem_t, 128, 128, 2, 2, AK, BK, MODE_PLAIN>;
    case CFG_DUAL: return gemm_kernel<elem_t, 128, 64, 2, 2, AK, BK, MODE_DUAL>;
    case CFG_PRO:
#if MI_TA == 0
      return gemm_kernel<elem_t, 128, 128, 2, 2, AK, BK, MODE_PROLOGUE>;
#else
      return nullptr;
#endif
  }
#endif
  return nullptr;
}

}  // namespace mig
