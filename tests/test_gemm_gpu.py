"""GPU parity of the HIP GEMM core against the CPU oracle, through the C ABI.

Bar: fp32 inputs within max relative error 1e-4, bf16 inputs within 1e-2 of the
float64 oracle fed the same bf16-rounded inputs (max relative error =
max|y - ref| / max|ref|). Small integers give bit-exact expectations. Full-size
benchmark configurations are checked on sampled rows against the oracle and on
every element through row/column checksums.
"""
import numpy as np
import pytest

from gpu_cases import (TOL_BF16, TOL_F32, check, checksums, host, inputs, layout, sample_rows,
                       to_dev)

pytestmark = pytest.mark.gpu


def _tol(bf16):
    return TOL_BF16 if bf16 else TOL_F32


def _run(mi, dev, oracle, M, N, K, tA, tB, bf16, seed, *, out_bf16=None, alpha=1.0, beta=0.0,
         bias=False, residual=False, dual=False, prologue=False, pad=(0, 0, 0), ws=None,
         a_std=1.0, b_std=0.02):
    import torch

    out_bf16 = bf16 if out_bf16 is None else out_bf16
    a = inputs(oracle, (M, K), seed, a_std, bf16)
    b = inputs(oracle, (K, N), seed + 1, b_std, bf16)
    A = layout(a, tA)
    B = layout(b, tB)
    lda, ldb, ldc = A.shape[1] + pad[0], B.shape[1] + pad[1], N + pad[2]
    Ap = np.zeros((A.shape[0], lda), np.float32); Ap[:, :A.shape[1]] = A
    Bp = np.zeros((B.shape[0], ldb), np.float32); Bp[:, :B.shape[1]] = B
    kw = {}
    ref_kw = {}
    if bias:
        bv = inputs(oracle, (N,), seed + 2, 0.02, bf16)
        kw["bias"] = to_dev(bv, dev, bf16)
        ref_kw["bias"] = bv
    c0 = inputs(oracle, (M, N), seed + 3, 0.5, out_bf16)
    C0 = np.zeros((M, ldc), np.float32); C0[:, :N] = c0
    if beta != 0.0:
        ref_kw.update(beta=beta, C0=c0)
    if residual:
        rv = inputs(oracle, (M, N), seed + 4, 0.5, bf16)
        kw["residual"] = to_dev(rv, dev, bf16)
        ref_kw["R"] = rv
    mode = 0
    if dual:
        b2 = inputs(oracle, (K, N), seed + 5, b_std, bf16)
        B2 = layout(b2, tB)
        B2p = np.zeros_like(Bp); B2p[:, :B2.shape[1]] = B2
        kw["B2"] = to_dev(B2p, dev, bf16)
        ref_kw["B2"] = b2
        mode = 1
    if prologue:
        a2 = inputs(oracle, (M, K), seed + 6, 1.0, bf16)
        A2p = np.zeros_like(Ap); A2p[:, :K] = a2
        kw["A2"] = to_dev(A2p, dev, bf16)
        ref_kw["A2"] = a2
        mode = 2
    C = to_dev(C0, dev, out_bf16)
    mi.gemm(to_dev(Ap, dev, bf16), to_dev(Bp, dev, bf16), C, M, N, K, transA=tA, transB=tB,
            alpha=alpha, beta=beta, lda=lda, ldb=ldb, ldc=ldc, workspace=ws, **kw)
    torch.cuda.synchronize()
    got = host(C)[:, :N]
    ref = oracle.gemm(0, 0, M, N, K, a, b, alpha=alpha, mode=mode, **ref_kw)
    return got, ref


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "f32"])
@pytest.mark.parametrize("tA,tB", [(0, 0), (0, 1), (1, 0), (1, 1)], ids=["NN", "NT", "TN", "TT"])
@pytest.mark.parametrize("shape", [(77, 130, 95), (320, 384, 256), (1, 1, 1), (5, 300, 17),
                                   (513, 257, 136)])
def test_layouts(mi, dev, oracle, bf16, tA, tB, shape):
    M, N, K = shape
    got, ref = _run(mi, dev, oracle, M, N, K, tA, tB, bf16, seed=100 + M)
    check(got, ref, _tol(bf16), f"{shape} tA={tA} tB={tB}")


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "f32"])
def test_leading_dimension_padding(mi, dev, oracle, bf16):
    for tA, tB in [(0, 0), (1, 1), (0, 1), (1, 0)]:
        got, ref = _run(mi, dev, oracle, 200, 136, 72, tA, tB, bf16, seed=7, pad=(8, 16, 4))
        check(got, ref, _tol(bf16), f"padded tA={tA} tB={tB}")
    # leading dimensions that break 16-byte alignment take the element-wise path
    got, ref = _run(mi, dev, oracle, 64, 40, 48, 0, 0, bf16, seed=8, pad=(3, 1, 1))
    check(got, ref, _tol(bf16), "unaligned ld")


def test_small_integers_bit_exact(mi, dev, oracle):
    """Integers in [-8, 8]: exact in bf16, sums exact in fp32 -> bit-exact outputs."""
    import torch

    rng = np.random.default_rng(5)
    for (M, N, K), (tA, tB) in [((300, 260, 520), (0, 0)), ((64, 96, 1000), (1, 0)),
                                ((129, 65, 33), (0, 1)), ((256, 256, 512), (1, 1))]:
        a = rng.integers(-8, 9, (M, K)).astype(np.float32)
        b = rng.integers(-8, 9, (K, N)).astype(np.float32)
        for bf16 in (True, False):
            C = torch.zeros((M, N), dtype=torch.float32, device=dev)
            mi.gemm(to_dev(layout(a, tA), dev, bf16), to_dev(layout(b, tB), dev, bf16), C, M, N, K,
                    transA=tA, transB=tB)
            assert np.array_equal(C.cpu().numpy(), a.astype(np.int64) @ b.astype(np.int64))


def test_bf16_output_rounds_to_nearest_even(mi, dev, oracle):
    """bf16 outputs whose exact fp32 values sit on rounding ties (1 + odd multiples
    of 2^-8 and their negatives) and off them: every output bit must equal the
    oracle's round-to-nearest-even (mo_f32_to_bf16_rne).  Tile-aligned shapes take
    the direct epilogue, an odd shape the general one; the beta = 1 pass adds a
    bf16 C read."""
    import torch

    deltas = np.array([1, 3, 5, 7, 2, 0.5, 1.5, -1, -3, 9, 11, 13], np.float32) * 2.0 ** -8
    for (M, N, K), (tA, tB) in [((512, 512, 64), (0, 1)), ((512, 256, 128), (0, 0)),
                                ((256, 512, 64), (1, 0)), ((130, 70, 40), (0, 1))]:
        a = np.zeros((M, K), np.float32)
        a[:, 0] = np.where(np.arange(M) % 2 == 0, 1.0, -1.0)
        a[:, 1] = deltas[np.arange(M) % len(deltas)]
        b = np.zeros((K, N), np.float32)
        b[0, :] = 1.0
        b[1, :] = np.array([1.0, 2.0, 0.5, 4.0], np.float32)[np.arange(N) % 4]
        exact = a.astype(np.float64) @ b.astype(np.float64)  # fp32-exact sums
        for beta in (0.0, 1.0):
            c0 = np.zeros((M, N), np.float32) if beta == 0.0 else oracle.round_bf16(exact)
            C = to_dev(c0, dev, True)
            mi.gemm(to_dev(layout(a, tA), dev, True), to_dev(layout(b, tB), dev, True), C, M, N, K,
                    transA=tA, transB=tB, beta=beta)
            want = oracle.to_bf16((exact + beta * c0.astype(np.float64)).astype(np.float32))
            got = C.view(torch.int16).cpu().numpy().view(np.uint16)
            assert np.array_equal(got, want), f"{M}x{N}x{K} tA={tA} tB={tB} beta={beta}"


def test_config1_fp32_linear_bias(mi, dev, oracle):
    """Benchmark configuration 1: Y = X W^T + b, X [512x768], W [768x768] ~ N(0,0.02), fp32."""
    import torch

    got, ref = _run(mi, dev, oracle, 512, 768, 768, 0, 1, False, seed=1, bias=True)
    check(got, ref, TOL_F32, "config 1")
    assert oracle.l2_rel_err(got, ref) < 1e-4  # test_gpu_kernels.cpp:87-116 metric
    # with the workspace the bridges pass, the same problem runs as split-K 5 (48 tiles of
    # 64x128)
    ws = torch.empty(mi.workspace_size(0, 1, 512, 768, 768, mi.MI_F32) // 4, dtype=torch.float32,
                     device=dev)
    assert _split_of(mi, 0, 1, 512, 768, 768, False, ws) == 5
    got, ref = _run(mi, dev, oracle, 512, 768, 768, 0, 1, False, seed=1, bias=True, ws=ws)
    check(got, ref, TOL_F32, "config 1, split-K")
    assert oracle.l2_rel_err(got, ref) < 1e-4


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "f32"])
def test_epilogues(mi, dev, oracle, bf16):
    for kw in [dict(bias=True), dict(beta=1.0), dict(beta=-0.5, alpha=2.0), dict(residual=True),
               dict(bias=True, beta=1.0, residual=True, alpha=0.5)]:
        for tA, tB in [(0, 0), (1, 0), (0, 1)]:
            got, ref = _run(mi, dev, oracle, 264, 200, 144, tA, tB, bf16, seed=21, **kw)
            check(got, ref, _tol(bf16), f"{kw} tA={tA} tB={tB}")
    # bf16 inputs with an fp32 output (dW) accumulating into the existing value
    got, ref = _run(mi, dev, oracle, 256, 320, 512, 1, 0, True, seed=22, out_bf16=False, beta=1.0)
    check(got, ref, TOL_BF16, "bf16 in / fp32 out, beta=1")


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "f32"])
def test_dual_silu_gate(mi, dev, oracle, bf16):
    """gemm_ffn: C = SiLU(A Bg) * (A Bu) (gemm_ffn.metal:160-181)."""
    for (M, N, K), (tA, tB) in [((300, 200, 160), (0, 0)), ((512, 384, 256), (0, 1)),
                                ((96, 72, 40), (1, 0))]:
        got, ref = _run(mi, dev, oracle, M, N, K, tA, tB, bf16, seed=31, dual=True, b_std=0.1)
        check(got, ref, _tol(bf16), f"dual {M}x{N}x{K}")


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "f32"])
def test_prologue_silu_gate(mi, dev, oracle, bf16):
    """fused_swiglu_gemm: C = (SiLU(G) * U) B (fused_swiglu_gemm.metal:48-77)."""
    for (M, N, K), tB in [((300, 200, 160), 0), ((512, 256, 512), 1), ((33, 17, 24), 0)]:
        got, ref = _run(mi, dev, oracle, M, N, K, 0, tB, bf16, seed=41, prologue=True)
        check(got, ref, _tol(bf16), f"prologue {M}x{N}x{K}")


def test_prologue_two_pass(mi, dev, oracle):
    """bf16 SiLU-gate prologue with a workspace for SiLU(G) * U: one activation pass,
    then the plain GEMM on it (the rest of the workspace left for its split-K).
    Shapes: a full-tile NN and NT case, edge tiles with padded leading dimensions,
    and a K that is not a multiple of 8 (in-load prologue, the workspace unused)."""
    import torch

    ws = torch.empty(8 << 20, dtype=torch.float32, device=dev)
    for (M, N, K), tB, pad in [((512, 512, 512), 0, (0, 0, 0)), ((512, 256, 1024), 1, (0, 0, 0)),
                               ((300, 200, 160), 0, (8, 4, 2)), ((64, 96, 100), 0, (0, 0, 0))]:
        got, ref = _run(mi, dev, oracle, M, N, K, 0, tB, True, seed=43, prologue=True, pad=pad,
                        ws=ws)
        check(got, ref, TOL_BF16, f"two-pass prologue {M}x{N}x{K} tB={tB}")


def test_fused_swiglu_gemm_config3_down(mi, dev, oracle):
    """The reference-named fused_swiglu_gemm at configuration 3's down projection
    (8192 x 2048, K = 5632): sampled rows against the oracle's SiLU-gate product and
    the column / row checksums of (SiLU(G) * U) W."""
    import torch

    M, N, K = 8192, 2048, 5632
    g = inputs(oracle, (M, K), 61, 1.0)
    u = inputs(oracle, (M, K), 62, 1.0)
    w = inputs(oracle, (K, N), 63, 0.02)
    G, U, W = to_dev(g, dev, True), to_dev(u, dev, True), to_dev(w, dev, True)
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    mi.fused_swiglu_gemm(G, U, W, C, M, N, K)
    torch.cuda.synchronize()
    rows = sample_rows(M, 6, 61)
    got = host(C)
    check(got[rows], oracle.gemm(0, 0, M, N, K, g, w, mode=2, A2=u, rows=rows), TOL_BF16, "down fwd rows")
    act = oracle.round_bf16((g / (1.0 + np.exp(-g.astype(np.float64)))) * u)
    col, row = checksums(act, w)
    check(got.sum(axis=0), col, TOL_BF16, "down fwd column checksum")
    check(got.sum(axis=1), row, TOL_BF16, "down fwd row checksum")


def _split_of(mi, tA, tB, M, N, K, bf16, ws):
    text = mi.describe(tA, tB, M, N, K, mi.MI_BF16 if bf16 else mi.MI_F32,
                       workspace_bytes=ws.numel() * 4)
    return int(text.split("split")[1].split()[0])


def test_split_k(mi, dev, oracle):
    """Split-K over the caller's workspace (partials + splitk_reduce_kernel): every case
    must plan a split above 1. TN dW forms with fp32 beta = 0 / 1 output, NN and NT
    forms, a register-staged case (leading dimensions that rule out 16-byte loads)
    and the bias + beta epilogue, which the reduction applies."""
    import torch

    ws = torch.empty(64 << 20, dtype=torch.float32, device=dev)
    cases = [
        dict(M=1024, N=1024, K=65536, tA=1, tB=0, beta=0.0),
        dict(M=256, N=384, K=30000, tA=1, tB=0, beta=1.0),
        dict(M=100, N=60, K=70000, tA=1, tB=0, beta=0.0),
        dict(M=512, N=256, K=20000, tA=0, tB=0, beta=0.0, out_bf16=True),
        dict(M=384, N=256, K=20000, tA=0, tB=1, beta=0.0, out_bf16=True),
        dict(M=200, N=136, K=20000, tA=0, tB=0, beta=0.5, bias=True, pad=(3, 1, 4)),
        dict(M=256, N=200, K=16384, tA=1, tB=0, beta=1.0, bias=True, alpha=0.5),
    ]
    for c in cases:
        M, N, K, tA, tB = c.pop("M"), c.pop("N"), c.pop("K"), c.pop("tA"), c.pop("tB")
        out_bf16 = c.pop("out_bf16", False)
        assert _split_of(mi, tA, tB, M, N, K, True, ws) > 1, (M, N, K, tA, tB)
        got, ref = _run(mi, dev, oracle, M, N, K, tA, tB, True, seed=51, out_bf16=out_bf16, ws=ws,
                        **c)
        check(got, ref, TOL_BF16, f"split-K {M}x{N}x{K} tA={tA} tB={tB} {c}")


def test_fp32_split_k(mi, dev, oracle):
    """fp32 split plans of configurations 1 and 2 and longer-K shapes (direct-to-LDS
    64x128 and 64x64 kernels writing partials, then the reduction) against the oracle
    at the fp32 bar."""
    import torch

    ws = torch.empty(16 << 20, dtype=torch.float32, device=dev)
    for (M, N, K), (tA, tB), kw in [((512, 768, 768), (0, 1), dict(bias=True)),
                                    ((768, 768, 2048), (1, 0), dict(beta=1.0)),
                                    ((2048, 768, 2304), (0, 1), {}),
                                    ((768, 1536, 4096), (1, 0), dict(beta=1.0, bias=True)),
                                    ((640, 2304, 4096), (1, 0), dict(beta=1.0)),
                                    ((1024, 768, 4096), (0, 0), dict(residual=True))]:
        assert _split_of(mi, tA, tB, M, N, K, False, ws) > 1, (M, N, K)
        got, ref = _run(mi, dev, oracle, M, N, K, tA, tB, False, seed=57, ws=ws, **kw)
        check(got, ref, TOL_F32, f"fp32 split-K {M}x{N}x{K} tA={tA} tB={tB} {kw}")
        assert oracle.l2_rel_err(got, ref) < 1e-4


@pytest.mark.parametrize("tA,tB", [(0, 0), (0, 1), (1, 0), (1, 1)], ids=["NN", "NT", "TN", "TT"])
def test_wave_split_k(mi, dev, oracle, tA, tB):
    """128x128 tiles with wave-level split-K (two groups of 4 waves, each over half of
    every K tile, summed through LDS): full tiles (direct epilogue), edge tiles with
    bias + residual (general epilogue), a K tail, fp32 beta = 1 output, and
    small-integer operands, whose outputs must be bit-exact."""
    import torch

    cases = [((256, 384, 2048), {}), ((384, 256, 1096), dict(beta=1.0, out_bf16=False)),
             ((200, 136, 1536), dict(bias=True, residual=True, alpha=0.5)),
             ((512, 512, 4096), dict(beta=-0.5, out_bf16=True))]
    for (M, N, K), kw in cases:
        assert "dlds-kg2" in mi.describe(tA, tB, M, N, K), (M, N, K)
        got, ref = _run(mi, dev, oracle, M, N, K, tA, tB, True, seed=71 + K, **kw)
        check(got, ref, TOL_BF16, f"wave split-K {M}x{N}x{K} tA={tA} tB={tB} {kw}")
    rng = np.random.default_rng(7)
    M, N, K = 384, 256, 2048
    a = rng.integers(-4, 5, (M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (K, N)).astype(np.float32)
    C = torch.zeros((M, N), dtype=torch.float32, device=dev)
    mi.gemm(to_dev(layout(a, tA), dev, True), to_dev(layout(b, tB), dev, True), C, M, N, K,
            transA=tA, transB=tB)
    assert np.array_equal(C.cpu().numpy(), a.astype(np.int64) @ b.astype(np.int64))


@pytest.mark.parametrize("tA,tB", [(0, 0), (0, 1), (1, 0), (1, 1)], ids=["NN", "NT", "TN", "TT"])
def test_fp32_direct_to_lds(mi, dev, oracle, tA, tB):
    """fp32 direct-to-LDS kernels, 64x128 and 64x64 tiles (K tile 32 of 128-byte rows,
    fp32 k-rows of a row-contiguous operand read 32 columns per half-wave): full tiles
    (direct epilogue, fp32 and bf16 C, beta), edge tiles with bias + residual (general
    epilogue), K tails, split-K partials, and small integers, whose outputs must be
    bit-exact."""
    import torch

    ws = torch.empty(16 << 20, dtype=torch.float32, device=dev)
    cases = [((2048, 2304, 768), {}, "64x64 "), ((2048, 768, 768), dict(beta=1.0), "64x128 "),
             ((256, 512, 132), dict(out_bf16=True), ""), ((200, 196, 100), dict(bias=True, residual=True), ""),
             ((320, 384, 256), dict(beta=-0.5, alpha=2.0, out_bf16=True), ""),
             ((384, 768, 2048), dict(beta=0.5), "split")]
    for (M, N, K), kw, want in cases:
        plan = mi.describe(tA, tB, M, N, K, mi.MI_F32, workspace_bytes=ws.numel() * 4)
        assert plan.startswith("dlds f32") and want in plan, plan
        got, ref = _run(mi, dev, oracle, M, N, K, tA, tB, False, seed=81 + K, ws=ws, **kw)
        # a bf16 C carries its own rounding (2^-9 relative)
        tol = TOL_BF16 if kw.get("out_bf16") else TOL_F32
        check(got, ref, tol, f"fp32 direct-to-LDS {M}x{N}x{K} tA={tA} tB={tB} {kw}")
    rng = np.random.default_rng(9)
    for (M, N, K) in [(384, 256, 1000), (256, 640, 96)]:
        a = rng.integers(-8, 9, (M, K)).astype(np.float32)
        b = rng.integers(-8, 9, (K, N)).astype(np.float32)
        C = torch.zeros((M, N), dtype=torch.float32, device=dev)
        assert mi.describe(tA, tB, M, N, K, mi.MI_F32).startswith("dlds f32")
        mi.gemm(to_dev(layout(a, tA), dev, False), to_dev(layout(b, tB), dev, False), C, M, N, K,
                transA=tA, transB=tB)
        assert np.array_equal(C.cpu().numpy(), a.astype(np.int64) @ b.astype(np.int64)), (M, N, K)


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "f32"])
@pytest.mark.parametrize("tA,tB", [(0, 0), (0, 1), (1, 0), (1, 1)], ids=["NN", "NT", "TN", "TT"])
def test_batched_head_groups(mi, dev, oracle, bf16, tA, tB):
    """mi_gemm_batched with a head map (batch x heads problems, B shared by groups of 2
    heads, as GQA's K/V) and with two K segments (C = sum over segments of A_s B_s), on
    the direct-to-LDS kernels (16-byte-aligned operands), against the oracle per problem."""
    import torch

    nb, heads, grp, M, N, K = 2, 4, 2, 136, 200, 136
    tol = _tol(bf16)
    a = inputs(oracle, (nb, heads, M, K), 61, 1.0, bf16)
    b = inputs(oracle, (nb, heads // grp, K, N), 62, 0.02, bf16)
    A = np.stack([np.stack([layout(a[i, h], tA) for h in range(heads)]) for i in range(nb)])
    B = np.stack([np.stack([layout(b[i, h], tB) for h in range(heads // grp)]) for i in range(nb)])
    C = torch.zeros((nb, heads, M, N), dtype=torch.float32, device=dev)
    bt = mi.make_batch(nb * heads, heads, a=(heads * M * K, M * K, 1),
                       b=((heads // grp) * K * N, K * N, grp), c=(heads * M * N, M * N, 1))
    assert mi.describe(tA, tB, M, N, K, mi.MI_BF16 if bf16 else mi.MI_F32,
                       batch=nb * heads).split()[0].startswith("dlds")
    mi.gemm_batched(to_dev(A, dev, bf16), to_dev(B, dev, bf16), C, M, N, K, bt, transA=tA, transB=tB)
    got = host(C)
    for i in range(nb):
        for h in range(heads):
            check(got[i, h], oracle.gemm(0, 0, M, N, K, a[i, h], b[i, h // grp]), tol,
                  f"problem ({i}, {h}) tA={tA} tB={tB}")
    # two K segments of one problem: C = A_0 B_0 + A_1 B_1 (segment strides in elements)
    C2 = torch.zeros((M, N), dtype=torch.float32, device=dev)
    seg_a, seg_b = M * K, K * N
    bt2 = mi.make_batch(1, 1, k_segments=2, seg_a=seg_a, seg_b=seg_b)
    mi.gemm_batched(to_dev(A[0, :2], dev, bf16), to_dev(B[0], dev, bf16), C2, M, N, K, bt2,
                    transA=tA, transB=tB)
    ref = oracle.gemm(0, 0, M, N, K, a[0, 0], b[0, 0]) + oracle.gemm(0, 0, M, N, K, a[0, 1], b[0, 1])
    check(host(C2), ref, tol, f"two K segments tA={tA} tB={tB}")


@pytest.mark.parametrize("tA,tB", [(0, 0), (0, 1), (1, 0), (1, 1)], ids=["NN", "NT", "TN", "TT"])
def test_tile_256x192(mi, dev, oracle, tA, tB):
    """256x192 tiles (8 waves of 64x96; a row-contiguous B stored in 128-byte granules
    of 64 columns): the direct epilogue, a K tail, and the bias epilogue. Sampled rows
    against the oracle, every element through checksums."""
    import torch

    M, N = 8192, 3072
    for K, bias in [(2048, False), (2000, False), (512, True)]:
        plan = mi.describe(tA, tB, M, N, K)
        assert "256x192" in plan, plan
        a = inputs(oracle, (M, K), 95 + K, 1.0)
        b = inputs(oracle, (K, N), 96 + K, 0.02)
        bv = inputs(oracle, (N,), 97, 0.02) if bias else None
        C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        extra = {"bias": torch.from_numpy(bv).to(dev)} if bias else {}
        mi.gemm(to_dev(layout(a, tA), dev, True), to_dev(layout(b, tB), dev, True), C, M, N, K,
                transA=tA, transB=tB, **extra)
        torch.cuda.synchronize()
        got = host(C)
        rows = sample_rows(M, 6, K)
        check(got[rows], oracle.gemm(0, 0, M, N, K, a, b, rows=rows, bias=bv), TOL_BF16,
              f"256x192 K={K} rows")
        col, row = checksums(a, b)
        if bias:
            col = col + M * bv.astype(np.float64)
            row = row + bv.astype(np.float64).sum()
        check(got.sum(axis=0), col, TOL_BF16, f"256x192 K={K} column checksum")
        check(got.sum(axis=1), row, TOL_BF16, f"256x192 K={K} row checksum")


@pytest.mark.parametrize("tA,tB", [(0, 0), (0, 1), (1, 0), (1, 1)], ids=["NN", "NT", "TN", "TT"])
def test_tile_128x192_split_k_groups(mi, dev, oracle, tA, tB):
    """128x192 tiles with wave-level split-K (two groups of 4 waves over halves of every
    K tile, summed through LDS; the qkv dW grid 2048x3072 in one round of 256 tiles):
    bf16 output, and fp32 beta = 1 accumulation. Sampled rows against the oracle, every
    element through checksums."""
    import torch

    M, N, K = 2048, 3072, 1024
    plan = mi.describe(tA, tB, M, N, K)
    assert "dlds-kg2 bf16 128x192" in plan, plan
    a = inputs(oracle, (M, K), 151 + 2 * tA + tB, 1.0)
    b = inputs(oracle, (K, N), 152 + 2 * tA + tB, 1e-2)
    rows = sample_rows(M, 6, 7)
    col, row = checksums(a, b)
    A, B = to_dev(layout(a, tA), dev, True), to_dev(layout(b, tB), dev, True)
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    mi.gemm(A, B, C, M, N, K, transA=tA, transB=tB)
    torch.cuda.synchronize()
    got = host(C)
    ref_rows = oracle.gemm(0, 0, M, N, K, a, b, rows=rows)
    check(got[rows], ref_rows, TOL_BF16, f"128x192 kg2 tA={tA} tB={tB} rows")
    check(got.sum(axis=0), col, TOL_BF16, f"128x192 kg2 tA={tA} tB={tB} column checksum")
    check(got.sum(axis=1), row, TOL_BF16, f"128x192 kg2 tA={tA} tB={tB} row checksum")
    c0 = inputs(oracle, (M, N), 153, 0.5, False)
    C32 = torch.from_numpy(c0).to(dev)
    mi.gemm(A, B, C32, M, N, K, transA=tA, transB=tB, beta=1.0)
    torch.cuda.synchronize()
    got = C32.cpu().numpy().astype(np.float64) - c0.astype(np.float64)
    check(got[rows], ref_rows, TOL_F32, f"128x192 kg2 tA={tA} tB={tB} beta=1 rows")
    check(got.sum(axis=0), col, TOL_F32, f"128x192 kg2 tA={tA} tB={tB} beta=1 column checksum")


def test_tile_256x192_partial_round(mi, dev, oracle):
    """256x192 tiles for a grid below one round of 256x256 tiles (the dW shapes of
    gate / up and down: 240 or 242 tiles instead of 176), TN with fp32 beta = 1
    accumulation, and N not a multiple of 192 (a last column tile of 64 or 128
    columns). Sampled rows against the oracle, every element through checksums."""
    import torch

    K = 1024
    for M, N in [(2048, 5632), (5632, 2048)]:
        plan = mi.describe(1, 0, M, N, K)
        assert "256x192 TN" in plan, plan
        a = inputs(oracle, (M, K), 131 + M, 1.0)
        b = inputs(oracle, (K, N), 132 + M, 1e-2)
        c0 = inputs(oracle, (M, N), 133 + M, 0.5, False)
        C = torch.from_numpy(c0).to(dev)
        mi.gemm(to_dev(layout(a, 1), dev, True), to_dev(b, dev, True), C, M, N, K, transA=True,
                beta=1.0)
        torch.cuda.synchronize()
        got = C.cpu().numpy().astype(np.float64) - c0.astype(np.float64)
        rows = sample_rows(M, 6, M)
        check(got[rows], oracle.gemm(0, 0, M, N, K, a, b, rows=rows), TOL_F32,
              f"256x192 TN {M}x{N} rows")
        col, row = checksums(a, b)
        check(got.sum(axis=0), col, TOL_F32, f"256x192 TN {M}x{N} column checksum")
        check(got.sum(axis=1), row, TOL_F32, f"256x192 TN {M}x{N} row checksum")


@pytest.mark.parametrize("out_bf16", [True, False], ids=["bf16_out", "f32_out"])
def test_direct_epilogue_edge_tiles(mi, dev, oracle, out_bf16):
    """M and N multiples of 32 but not of the tile: the direct epilogue stores the edge
    tiles' 32x32 blocks inside the matrix and skips the rest (with beta * C read back)."""
    for i, (M, N, K, tA, tB) in enumerate([(288, 416, 512, 0, 0), (1056, 800, 1024, 0, 1),
                                           (512, 1120, 1024, 1, 0), (2080, 2272, 256, 0, 0)]):
        got, ref = _run(mi, dev, oracle, M, N, K, tA, tB, True, seed=141 + i, out_bf16=out_bf16,
                        beta=0.5)
        check(got, ref, TOL_BF16, f"edge tiles {M}x{N}x{K} tA={tA} tB={tB}")


def test_zero_k(mi, dev, oracle):
    got, ref = _run(mi, dev, oracle, 70, 90, 0, 0, 0, False, seed=61, beta=0.5, bias=True)
    check(got, ref, TOL_F32, "K=0")


# ---- decoder-block GEMM sets of the benchmark configurations ----------------------

def _block_set(mi, dev, oracle, M, H, Nqkv, I, bf16, seed, ws=None):
    """Forward (NN), dX (NT) and dW (TN) for QKV, O, gate, up, down: engine layout W[in,out].
    Returns the largest split-K factor the 15 products planned."""
    import torch

    shapes = {"qkv": (H, Nqkv), "o": (H, H), "gate": (H, I), "up": (H, I), "down": (I, H)}
    rows = sample_rows(M, 6, seed)
    max_split = 1
    for name, (din, dout) in shapes.items():
        x = inputs(oracle, (M, din), seed + 1, 1.0, bf16)
        w = inputs(oracle, (din, dout), seed + 2, 0.02, bf16)
        dy = inputs(oracle, (M, dout), seed + 3, 1e-2, bf16)
        X, W, dY = to_dev(x, dev, bf16), to_dev(w, dev, bf16), to_dev(dy, dev, bf16)
        odt = torch.bfloat16 if bf16 else torch.float32
        Y = torch.empty((M, dout), dtype=odt, device=dev)
        dX = torch.empty((M, din), dtype=odt, device=dev)
        dW = torch.zeros((din, dout), dtype=torch.float32, device=dev)
        mi.gemm(X, W, Y, M, dout, din, workspace=ws)                    # Y = X W
        mi.gemm(dY, W, dX, M, din, dout, transB=True, workspace=ws)     # dX = dY W^T
        mi.gemm(X, dY, dW, din, dout, M, transA=True, beta=1.0, workspace=ws)  # dW += X^T dY
        if ws is not None:
            max_split = max([max_split] + [_split_of(mi, *f, bf16, ws) for f in
                                           [(0, 0, M, dout, din), (0, 1, M, din, dout),
                                            (1, 0, din, dout, M)]])
        torch.cuda.synchronize()
        tol = TOL_BF16 if bf16 else TOL_F32
        y, dx, dw = host(Y), host(dX), host(dW)
        check(y[rows], oracle.gemm(0, 0, M, dout, din, x, w, rows=rows), tol, f"{name} fwd")
        check(dx[rows], oracle.gemm(0, 1, M, din, dout, dy, w, rows=rows), tol, f"{name} dX")
        wrows = sample_rows(din, 6, seed + 9)
        check(dw[wrows], oracle.gemm(1, 0, din, dout, M, x, dy, rows=wrows), tol, f"{name} dW")
        for got, (a_op, b_op) in [(y, (x, w)), (dx, (dy, w.T)), (dw, (x.T, dy))]:
            col, row = checksums(a_op, b_op)
            check(got.sum(axis=0), col, tol, f"{name} column checksum")
            check(got.sum(axis=1), row, tol, f"{name} row checksum")
    return max_split


@pytest.mark.parametrize("with_ws", [False, True], ids=["no_ws", "split_k"])
def test_config2_gpt_small_fp32(mi, dev, oracle, with_ws):
    """Benchmark configuration 2: d=768, 12 heads MHA (QKV 768->2304), SwiGLU 2048, M=2048, fp32.
    With the workspace the bridges pass, 8 of the 15 products run split-K (2, and 3 for
    o dW), over 64x64 tiles."""
    import torch

    ws = torch.empty(8 << 20, dtype=torch.float32, device=dev) if with_ws else None
    max_split = _block_set(mi, dev, oracle, 2048, 768, 2304, 2048, False, seed=200, ws=ws)
    assert max_split == (3 if with_ws else 1)


def test_config3_1p6b_bf16(mi, dev, oracle):
    """Benchmark configuration 3: d=2048, GQA 16/4 x 128 (QKV 2048->3072), SwiGLU 5632, M=8192, bf16."""
    _block_set(mi, dev, oracle, 8192, 2048, 3072, 5632, True, seed=300)


def test_config5_lm_head(mi, dev, oracle):
    """Benchmark configuration 5: logits = X E^T (NT), dX = dL E (NN), dE = dL^T X (TN, fp32)."""
    import torch

    M, H, V = 8192, 2048, 32000
    x = inputs(oracle, (M, H), 501, 1.0)
    e = inputs(oracle, (V, H), 502, 0.02)
    dl = inputs(oracle, (M, V), 503, 1e-3)
    X, E, dL = to_dev(x, dev, True), to_dev(e, dev, True), to_dev(dl, dev, True)
    logits = torch.empty((M, V), dtype=torch.bfloat16, device=dev)
    dX = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
    dE = torch.zeros((V, H), dtype=torch.float32, device=dev)
    mi.gemm(X, E, logits, M, V, H, transB=True)
    mi.gemm(dL, E, dX, M, H, V)
    mi.gemm(dL, X, dE, V, H, M, transA=True, beta=1.0)
    torch.cuda.synchronize()
    rows = sample_rows(M, 4, 5)
    check(host(logits[rows]), oracle.gemm(0, 1, M, V, H, x, e, rows=rows), TOL_BF16, "logits")
    check(host(dX[rows]), oracle.gemm(0, 0, M, H, V, dl, e, rows=rows), TOL_BF16, "dX")
    vrows = sample_rows(V, 4, 6)
    check(host(dE[vrows]), oracle.gemm(1, 0, V, H, M, dl, x, rows=vrows), TOL_BF16, "dE")
    for got, (a_op, b_op) in [(logits, (x, e.T)), (dX, (dl, e)), (dE, (dl.T, x))]:
        g = host(got)
        col, row = checksums(a_op, b_op)
        check(g.sum(axis=0), col, TOL_BF16, "column checksum")
        check(g.sum(axis=1), row, TOL_BF16, "row checksum")


# ---- per-call GEMM profiler ---------------------------------------------------------

def test_profiler_records_block_set(mi, dev, oracle):
    """GemmProfiler over configuration 3's 15 GEMMs: one record per call, in call
    order, with the call's shape and transposes, the plan mi_gemm_describe names for
    it and a positive GPU time; the totals add up the records."""
    import torch

    M, H, Nqkv, I = 8192, 2048, 3072, 5632
    shapes = [(H, Nqkv), (H, H), (H, I), (H, I), (I, H)]
    prof = mi.GemmProfiler.instance()
    prof.enable()
    try:
        prof.begin_step()
        mi.reset_profile_stats()
        want = []
        for din, dout in shapes:
            X = torch.randn((M, din), device=dev).to(torch.bfloat16)
            W = (0.02 * torch.randn((din, dout), device=dev)).to(torch.bfloat16)
            dY = (1e-2 * torch.randn((M, dout), device=dev)).to(torch.bfloat16)
            Y = torch.empty((M, dout), dtype=torch.bfloat16, device=dev)
            dX = torch.empty((M, din), dtype=torch.bfloat16, device=dev)
            dW = torch.zeros((din, dout), dtype=torch.float32, device=dev)
            mi.gemm(X, W, Y, M, dout, din, sync=False)
            mi.gemm(dY, W, dX, M, din, dout, transB=True, sync=False)
            mi.gemm(X, dY, dW, din, dout, M, transA=True, beta=1.0, sync=False)
            want += [(M, dout, din, False, False), (M, din, dout, False, True),
                     (din, dout, M, True, False)]
        recs = prof.records()
        assert len(recs) == 15
        for r, (m, n, k, ta, tb) in zip(recs, want):
            assert (r["M"], r["N"], r["K"], r["transA"], r["transB"]) == (m, n, k, ta, tb)
            assert r["kernel"] == mi.describe(ta, tb, m, n, k), r
            assert r["splits"] == 1 and r["batch"] == 1
            assert 0.0 < r["elapsed_ms"] < 100.0, r
        ms, calls = mi.accum_gpu_time_ms(), mi.count_gpu_calls()
        assert calls == 15
        assert abs(ms - sum(r["elapsed_ms"] for r in recs)) < 1e-6 * max(ms, 1.0) + 1e-9
        rows = prof.summary()
        assert sum(a["calls"] for a in rows) == 15
        prof.print_summary(ms)
        prof.begin_step()
        assert prof.records() == []
        assert mi.count_gpu_calls() == 15      # the totals survive begin_step
        mi.reset_profile_stats()
        assert mi.count_gpu_calls() == 0
    finally:
        prof.enable(False)
        prof.begin_step()
    # recording off: nothing is kept
    A = torch.zeros((64, 64), dtype=torch.bfloat16, device=dev)
    C = torch.empty((64, 64), dtype=torch.bfloat16, device=dev)
    mi.gemm(A, A, C, 64, 64, 64)
    assert prof.records() == []


# ---- Tensor::matmul mirror --------------------------------------------------------

@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "f32"])
def test_tensor_matmul_mirror(mi, dev, oracle, bf16):
    # TC-12 / TC-13 known answers (test_math_ops.cpp:167-189)
    A = to_dev(np.array([[1, 2, 3], [4, 5, 6]], np.float32), dev, bf16)
    B = to_dev(np.array([[7, 8], [9, 10], [11, 12]], np.float32), dev, bf16)
    assert host(mi.matmul(A, B)).tolist() == [[58, 64], [139, 154]]
    A3 = to_dev(np.array([1, 2, 3, 4, 5, 6, 1, 1, 1, 2, 2, 2], np.float32).reshape(2, 2, 3), dev,
                bf16)
    B3 = to_dev(np.array([7, 8, 9, 10, 11, 12, 1, 2, 3, 4, 5, 6], np.float32).reshape(2, 3, 2),
                dev, bf16)
    C3 = host(mi.matmul(A3, B3))
    assert C3[0, 0, 0] == 58 and C3[1, 1, 1] == 24
    # projection branch: [2, 96, 160] x [160, 72]
    x = inputs(oracle, (2, 96, 160), 71, 1.0, bf16)
    w = inputs(oracle, (160, 72), 72, 0.05, bf16)
    y = host(mi.matmul(to_dev(x, dev, bf16), to_dev(w, dev, bf16)))
    check(y.reshape(192, 72), oracle.gemm(0, 0, 192, 72, 160, x.reshape(192, 160), w), _tol(bf16))
    # batched branch: [2, 3, 40, 24] x [2, 3, 24, 56]
    a = inputs(oracle, (2, 3, 40, 24), 73, 1.0, bf16)
    b = inputs(oracle, (2, 3, 24, 56), 74, 1.0, bf16)
    c = host(mi.matmul(to_dev(a, dev, bf16), to_dev(b, dev, bf16)))
    for i in range(2):
        for j in range(3):
            check(c[i, j], oracle.gemm(0, 0, 40, 56, 24, a[i, j], b[i, j]), _tol(bf16))
    with pytest.raises(ValueError, match="Inner dimensions must match for projection"):
        mi.matmul(to_dev(x, dev, bf16), to_dev(x[0], dev, bf16))


def test_reference_named_entry_points(mi, dev, oracle):
    import torch

    M, N, K = 192, 160, 128
    a = inputs(oracle, (M, K), 81)
    b = inputs(oracle, (K, N), 82, 0.05)
    A, B = to_dev(a, dev, True), to_dev(b, dev, True)
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    mi.begin_scope()
    mi.gemm_bf16(A, B, C, M, N, K)
    mi.end_scope()
    check(host(C), oracle.gemm(0, 0, M, N, K, a, b), TOL_BF16, "gemm_bf16")
    Bt = to_dev(layout(b, 1), dev, True)
    mi.gemm_proj_trans_b(A, Bt, C, M, N, K)
    check(host(C), oracle.gemm(0, 0, M, N, K, a, b), TOL_BF16, "gemm_proj_trans_b")
    At = to_dev(layout(a, 1), dev, True)
    mi.gemm_backward(At, B, C, M, N, K)
    check(host(C), oracle.gemm(0, 0, M, N, K, a, b), TOL_BF16, "gemm_backward")
    D = torch.ones((M, N), dtype=torch.float32, device=dev)
    mi.gemm_backward(At, B, D, M, N, K, accumulate=True)
    check(host(D), oracle.gemm(0, 0, M, N, K, a, b) + 1.0, TOL_BF16, "gemm_backward +=")
    af, bf = inputs(oracle, (M, K), 83, bf16=False), inputs(oracle, (K, N), 84, 0.05, bf16=False)
    Cf = torch.empty((M, N), dtype=torch.float32, device=dev)
    mi.gemm_proj(to_dev(af, dev, False), to_dev(bf, dev, False), Cf, M, N, K)
    check(host(Cf), oracle.gemm(0, 0, M, N, K, af, bf), TOL_F32, "gemm_proj")
    R = torch.full((M, N), 0.25, dtype=torch.float32, device=dev)
    mi.residual_add(Cf, R)
    check(host(Cf), oracle.gemm(0, 0, M, N, K, af, bf) + 0.25, TOL_F32, "residual_add")
    mi.gemm_bf16(A, B, C, 0, N, K)  # zero-size no-op


def test_cpp_bridge_program():
    """The C++ mirror (include/gemm_bridge.hpp) run by tests/cpp/test_bridge."""
    import os
    import subprocess

    exe = os.path.join(os.path.dirname(__file__), "cpp", "test_bridge")
    assert os.path.exists(exe), "tests/cpp/test_bridge not built (run __graft_entry__.build())"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
