"""RMSNorm folded into the next GEMM (the survey's norm-prologue row): the decoder layer's
rmsnorm(h [+= residual]) @ W (Transformer.cpp:147-162, Attention.cpp:196-201) computed as
one row statistic and one GEMM on h itself,

    rmsnorm(h) W = diag(1/rms) h W',   W' = diag(weight) W,

with 1/rms the GEMM's epilogue row scale (mi_rmsnorm_fwd with y = NULL,
mi_rmsnorm_fold_weight, mi_gemm with epi->row_scale).

Checks: the statistic-only norm gives the full norm's rstd and residual sum bit for bit;
the folded weight equals numpy's RNE-rounded product bit for bit; the GEMM row scale against
the oracle with the rows of A pre-scaled in float64 (every kernel family: direct-to-LDS
fast and general epilogues, edge tiles, split-K, the fp32 register-staged kernel); and the
whole fold against the oracle's norm followed by its GEMM, at small sizes and at
configuration 3's QKV projection (8192 x 2048 -> 3072), with and without the residual add.
Tolerances: 1e-2 for bf16 inputs, 1e-4 for fp32 (max |got - ref| / max |ref|).
"""
import numpy as np
import pytest

from gpu_cases import TOL_BF16, TOL_F32, check, host, inputs, layout, sample_rows, to_dev

pytestmark = pytest.mark.gpu


def _rne_bf16(x):
    """float32 -> bf16 (round to nearest even) -> float32, numpy."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("rows,dims,dt", [(64, 2048, "bf16"), (33, 768, "f32"), (9, 100, "bf16")])
def test_statistic_only_matches_full_norm(mi, dev, rows, dims, dt):
    """y = NULL: the same rstd and the same stored residual sum as the full forward."""
    import torch

    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}[dt]
    g = torch.Generator(device=dev)
    g.manual_seed(rows + dims)
    x = torch.randn((rows, dims), generator=g, device=dev).to(tdt)
    r = (torch.randn((rows, dims), generator=g, device=dev) * 0.5).to(tdt)
    w = (1.0 + 0.2 * torch.randn((dims,), generator=g, device=dev)).to(tdt)
    for res in (None, r):
        x1, x2 = x.clone(), x.clone()
        s1 = torch.empty((rows,), dtype=torch.float32, device=dev)
        s2 = torch.empty_like(s1)
        mi.rms_norm_forward(x1, w, residual=res, rstd=s1)
        mi.rms_norm_forward(x2, w, residual=res, out=False, rstd=s2)
        assert torch.equal(s1, s2), "rstd differs from the full norm's"
        assert torch.equal(x1, x2), "residual sum differs from the full norm's"


@pytest.mark.parametrize("K,N,dt,wdt", [(2048, 3072, "bf16", "f32"), (768, 2304, "f32", "f32"),
                                        (96, 100, "bf16", "bf16"), (5, 7, "f32", "bf16")])
def test_fold_weight_exact(mi, dev, K, N, dt, wdt):
    """W'[k, n] = RNE(weight[k] * W[k, n]) bit for bit, vector and element paths, and in place."""
    import torch

    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}
    rng = np.random.default_rng(K + N)
    W = torch.from_numpy(rng.normal(0, 0.02, (K, N)).astype(np.float32)).to(dev, tdt[dt])
    w = torch.from_numpy(rng.normal(1, 0.2, K).astype(np.float32)).to(dev, tdt[wdt])
    got = mi.rms_norm_fold_weight(w, W)
    prod = (w.float().cpu().numpy()[:, None] * W.float().cpu().numpy()).astype(np.float32)
    want = _rne_bf16(prod) if dt == "bf16" else prod
    assert np.array_equal(got.float().cpu().numpy().view(np.uint32), want.view(np.uint32))
    inplace = W.clone()
    mi.rms_norm_fold_weight(w, inplace, out=inplace)
    assert torch.equal(inplace, got)


# (M, N, K, transA, transB, bf16, bias, beta, workspace bytes)
ROW_SCALE_CASES = [
    (512, 768, 512, 0, 0, True, False, 0.0, 0),            # 256x256 direct epilogue
    (8192 // 16, 3072, 2048, 0, 0, True, False, 0.0, 0),     # 256x192 tiles
    (300, 200, 256, 0, 1, True, True, 1.0, 0),              # edge tiles, bias, beta: general epilogue
    (256, 384, 20000, 1, 0, True, False, 0.0, 64 << 20),    # split-K + reduction kernel
    (384, 512, 768, 0, 0, False, True, 0.0, 0),             # fp32 register-staged kernel
    (96, 128, 4096, 0, 1, False, False, 0.0, 64 << 20),     # fp32 split-K
]


@pytest.mark.parametrize("case", range(len(ROW_SCALE_CASES)))
def test_gemm_row_scale(mi, dev, oracle, case):
    import torch

    M, N, K, tA, tB, bf16, bias, beta, wsb = ROW_SCALE_CASES[case]
    print(f"row scale M={M} N={N} K={K} tA={tA} tB={tB} bf16={bf16} bias={bias} beta={beta}", flush=True)
    a = inputs(oracle, (M, K), 700 + case, 1.0, bf16)
    b = inputs(oracle, (K, N), 701 + case, 0.02, bf16)
    s = np.random.default_rng(case).uniform(0.25, 4.0, M).astype(np.float32)
    c0 = inputs(oracle, (M, N), 702 + case, 0.5, False)
    bv = inputs(oracle, (N,), 703 + case, 0.1, False) if bias else None
    A, B = to_dev(layout(a, tA), dev, bf16), to_dev(layout(b, tB), dev, bf16)
    S = torch.from_numpy(s).to(dev)
    C = torch.from_numpy(c0).to(dev, torch.bfloat16 if bf16 and not beta else torch.float32)
    kw = {"bias": torch.from_numpy(bv).to(dev)} if bias else {}
    ws = torch.empty((wsb // 4,), dtype=torch.float32, device=dev) if wsb else None
    mi.gemm(A, B, C, M, N, K, transA=bool(tA), transB=bool(tB), beta=beta, row_scale=S,
            workspace=ws, **kw)
    # oracle: diag(s) (A B) in float64 (= (diag(s) A) B), then bias and beta * C0
    ref = oracle.gemm(0, 0, M, N, K, a, b) * s[:, None].astype(np.float64)
    if bias:
        ref = ref + bv[None, :]
    if beta:
        ref = ref + beta * c0
    check(host(C), ref, TOL_BF16 if bf16 else TOL_F32, "row-scaled GEMM")


@pytest.mark.parametrize("M,K,N,dt,res", [(300, 256, 384, "bf16", False), (256, 768, 2304, "f32", True),
                                          (512, 2048, 3072, "bf16", True)])
def test_rms_norm_matmul_vs_oracle(mi, dev, oracle, M, K, N, dt, res):
    """The fold against the oracle's norm (RMSNorm.cpp:40-75, residual add of
    Transformer.cpp:150-158) followed by its GEMM, and against the unfused library path."""
    import torch

    bf16 = dt == "bf16"
    tdt = torch.bfloat16 if bf16 else torch.float32
    x = inputs(oracle, (M, K), 810, 1.0, bf16)
    r = inputs(oracle, (M, K), 811, 0.5, bf16) if res else None
    w = inputs(oracle, (K,), 812, 0.2, False) + 1.0
    W = inputs(oracle, (K, N), 813, 0.02, bf16)
    X, Wt = to_dev(x, dev, bf16), to_dev(W, dev, bf16)
    Wn = torch.from_numpy(w.astype(np.float32)).to(dev)
    R = to_dev(r, dev, bf16) if res else None
    X2 = X.clone()
    C = mi.rms_norm_matmul(X, Wn, Wt, residual=R)
    y, _, x_after = oracle.rmsnorm_fwd(x, w, residual=r, round_bf16=bf16)
    ref = oracle.gemm(0, 0, M, N, K, y.astype(np.float64), W)
    check(host(C), ref, TOL_BF16 if bf16 else TOL_F32, "folded norm + GEMM vs oracle")
    if res:
        assert np.array_equal(X.float().cpu().numpy(), x_after), "x += residual as stored"
    # unfused: the norm kernel, then the GEMM on its output
    Y = torch.empty_like(X2)
    mi.rms_norm_forward(X2, Wn, residual=R, out=Y)
    C2 = torch.empty_like(C)
    mi.gemm(Y, Wt, C2, M, N, K)
    check(host(C), host(C2), 2 * (TOL_BF16 if bf16 else TOL_F32), "folded vs unfused")


def test_rms_norm_matmul_config3_qkv(mi, dev, oracle):
    """Configuration 3's attention input norm and QKV projection (8192 x 2048 -> 3072, bf16,
    residual add first): sampled rows against the oracle."""
    import torch

    M, K, N = 8192, 2048, 3072
    x = inputs(oracle, (M, K), 820, 1.0, True)
    r = inputs(oracle, (M, K), 821, 0.5, True)
    w = inputs(oracle, (K,), 822, 0.2, False) + 1.0
    W = inputs(oracle, (K, N), 823, 0.02, True)
    X, R, Wt = to_dev(x, dev, True), to_dev(r, dev, True), to_dev(W, dev, True)
    Wn = torch.from_numpy(w.astype(np.float32)).to(dev)
    C = host(mi.rms_norm_matmul(X, Wn, Wt, residual=R))
    rows = sample_rows(M, 8, 3)
    y, _, _ = oracle.rmsnorm_fwd(x[rows], w, residual=r[rows], round_bf16=True)
    ref = oracle.gemm(0, 0, len(rows), N, K, y.astype(np.float64), W)
    check(C[rows], ref, TOL_BF16, "configuration-3 QKV rows")
