"""mi_gemm_noalloc: the GEMM entry point that allocates nothing (split-K partials go
to the library's static per-GPU scratch array instead of a caller workspace).

Bar: its output equals, bit for bit, that of mi_gemm given a workspace of
mi_gemm_workspace_size bytes (same plan, same kernels, fixed-order split-K
reduction), and is within the north-star tolerance of the oracle. Each pair of
calls runs twice in a row, the second time on a smaller problem, so the second
call finds the first call's partials still in the scratch array. With the
SiLU-gate prologue (epi->A2) the comparison is mi_gemm given no workspace: both
then run the in-load prologue (the two-pass form needs an M x K activation
buffer that the scratch does not hold).
"""
import ctypes

import numpy as np
import pytest

from gpu_cases import TOL_BF16, TOL_F32, check, host, inputs, layout, sample_rows, to_dev

pytestmark = pytest.mark.gpu


def _dt(mi, t):
    import torch

    return mi.MI_BF16 if t.dtype == torch.bfloat16 else mi.MI_F32


def _problem(mi, dev, oracle, M, N, K, tA, tB, bf16, seed, beta, bias, gate=False):
    import torch

    a = inputs(oracle, (M, K), seed, 1.0, bf16)
    b = inputs(oracle, (K, N), seed + 1, 0.02, bf16)
    c0 = inputs(oracle, (M, N), seed + 2, 0.5, False)
    bv = inputs(oracle, (N,), seed + 3, 0.02, False) if bias else None
    u = inputs(oracle, (M, K), seed + 4, 1.0, bf16) if gate else None
    A, B = to_dev(layout(a, tA), dev, bf16), to_dev(layout(b, tB), dev, bf16)
    C0 = torch.from_numpy(c0).to(dev)
    rows = sample_rows(M, 8, seed) if M * N * K > (1 << 30) else np.arange(M)
    extra = {"A2": u, "mode": 2} if gate else {}
    ref = oracle.gemm(0, 0, M, N, K, a, b, rows=rows, **({"bias": bv} if bias else {}),
                      **({"beta": beta, "C0": c0} if beta else {}), **extra)
    epi = None
    keep = []
    if bias or gate:
        epi = mi.MiEpilogue()
    if bias:
        bt = torch.from_numpy(bv).to(dev)
        keep.append(bt)
        epi.bias, epi.bias_dtype = bt.data_ptr(), mi.MI_F32
    if gate:
        U = to_dev(u, dev, bf16)
        keep.append(U)
        epi.A2 = U.data_ptr()
    return A, B, C0, epi, (rows, ref), keep


def _call_noalloc(mi, A, B, C, M, N, K, tA, tB, beta, epi):
    L = mi.load_library()
    lda, ldb = (M if tA else K), (K if tB else N)
    return L.mi_gemm_noalloc(mi._stream(), tA, tB, M, N, K, 1.0, ctypes.c_void_p(A.data_ptr()), lda,
                             ctypes.c_void_p(B.data_ptr()), ldb, _dt(mi, A), beta,
                             ctypes.c_void_p(C.data_ptr()), N, _dt(mi, C),
                             ctypes.byref(epi) if epi is not None else None)


def _call_ws(mi, A, B, C, M, N, K, tA, tB, beta, epi, ws):
    L = mi.load_library()
    lda, ldb = (M if tA else K), (K if tB else N)
    wsp = ctypes.c_void_p(ws.data_ptr()) if ws is not None else None
    wsb = ws.numel() * 4 if ws is not None else 0
    return L.mi_gemm(mi._stream(), tA, tB, M, N, K, 1.0, ctypes.c_void_p(A.data_ptr()), lda,
                     ctypes.c_void_p(B.data_ptr()), ldb, _dt(mi, A), beta,
                     ctypes.c_void_p(C.data_ptr()), N, _dt(mi, C),
                     ctypes.byref(epi) if epi is not None else None, wsp, wsb)


SCRATCH_BYTES = 32 << 20  # MI_NOALLOC_SCRATCH_BYTES (include/mi_gemm.h)

# (M, N, K, tA, tB, bf16 inputs, beta, bias, SiLU-gate A2); each pair: larger problem,
# then smaller. The first problem of the first three pairs plans a split-K (asserted
# below), so the second call finds partials of the first in the scratch.
PAIRS = [
    # fp32 configuration 2 o dW, then configuration 1 (NT + bias)
    ((768, 768, 2048, 1, 0, False, 1.0, False, False), (512, 768, 768, 0, 1, False, 0.0, True, False)),
    # bf16 tall-K weight gradients, the second with beta = 1
    ((1024, 1024, 65536, 1, 0, True, 0.0, False, False),
     (256, 384, 30000, 1, 0, True, 1.0, False, False)),
    # a split NN problem with bias, then one without a split
    ((512, 256, 20000, 0, 0, True, 0.0, True, False), (1024, 768, 512, 0, 0, True, 0.0, False, False)),
    # SiLU-gate prologue (fused_swiglu_gemm): small N, long K (whose two-pass form would
    # need a 22 MiB activation), then a smaller problem with beta = 1
    ((2048, 512, 5632, 0, 0, True, 0.0, False, True), (256, 384, 1024, 0, 0, True, 1.0, False, True)),
]


@pytest.mark.parametrize("pair", range(len(PAIRS)))
def test_noalloc_matches_workspace_entry_point(mi, dev, oracle, pair):
    import torch

    for seed, (M, N, K, tA, tB, bf16, beta, bias, gate) in enumerate(PAIRS[pair]):
        print(f"noalloc case M={M} N={N} K={K} tA={tA} tB={tB} bf16={bf16} beta={beta} bias={bias} "
              f"gate={gate}", flush=True)
        dt_in = mi.MI_BF16 if bf16 else mi.MI_F32
        # the SiLU-gate prologue runs unsplit, as mi_gemm does without a workspace
        need = 0 if gate else mi.workspace_size(tA, tB, M, N, K, dt_in, mi.MI_F32)
        assert need <= SCRATCH_BYTES
        if seed == 0 and pair < 3:
            assert need > 0, "the first problem of the pair should plan a split-K"
        A, B, C0, epi, ref, keep = _problem(mi, dev, oracle, M, N, K, tA, tB, bf16, 900 + 10 * seed,
                                            beta, bias, gate)
        ws = torch.empty(max(need // 4, 1), dtype=torch.float32, device=dev) if need else None
        C_ws, C_na = C0.clone(), C0.clone()
        assert _call_ws(mi, A, B, C_ws, M, N, K, tA, tB, beta, epi, ws) == 0, \
            mi.load_library().mi_last_error()
        assert _call_noalloc(mi, A, B, C_na, M, N, K, tA, tB, beta, epi) == 0, \
            mi.load_library().mi_last_error()
        torch.cuda.synchronize()
        got_ws, got_na = C_ws.cpu().numpy(), C_na.cpu().numpy()
        assert np.array_equal(got_na.view(np.uint32), got_ws.view(np.uint32)), (M, N, K)
        rows, want = ref
        check(host(C_na)[rows], want, TOL_BF16 if bf16 else TOL_F32, f"noalloc {M}x{N}x{K}")
        del keep


def test_noalloc_validation(mi, dev):
    """Argument errors are reported like mi_gemm's; an empty output is a no-op."""
    import torch

    L = mi.load_library()
    A = torch.zeros((64, 64), dtype=torch.bfloat16, device=dev)
    p = ctypes.c_void_p(A.data_ptr())
    assert L.mi_gemm_noalloc(None, 0, 0, 64, 64, 64, 1.0, p, 10, p, 64, mi.MI_BF16, 0.0, p, 64,
                             mi.MI_BF16, None) == 2                               # MI_ERR_LD
    assert L.mi_gemm_noalloc(None, 0, 0, 64, 64, 64, 1.0, None, 64, p, 64, mi.MI_BF16, 0.0, p,
                             64, mi.MI_BF16, None) == 3                           # MI_ERR_NULL
    assert L.mi_gemm_noalloc(None, 0, 0, 0, 64, 64, 1.0, None, 64, None, 64, mi.MI_BF16, 0.0,
                             None, 64, mi.MI_BF16, None) == 0                     # no-op
