"""GQA attention batched GEMM forms on the GPU vs the oracle's restatement of
Attention.cpp:236-280 (forward) and 292-348 (backward), bf16 in / fp32 accumulate.

S = Q K^T / sqrt(d) (NT, kv-head map, causal output mask), softmax, O = P V (NN,
causal K skipping), dV = P^T dO and dK = dS^T Q (TN, K loop over the query heads
of a KV group = the KV-group reduction), dP = dO V^T (NT), dQ = dS K (NN).
"""
import numpy as np
import pytest

from gpu_cases import TOL_BF16, check, dense_attention, dense_attention_bwd, host, inputs, layout, to_dev

pytestmark = pytest.mark.gpu


def _qkv(oracle, Bn, nH, nKV, T, d, seed):
    q = inputs(oracle, (Bn, nH, T, d), seed)
    k = inputs(oracle, (Bn, nKV, T, d), seed + 1)
    v = inputs(oracle, (Bn, nKV, T, d), seed + 2)
    do = inputs(oracle, (Bn, T, nH * d), seed + 3, 1e-2)
    return q, k, v, do


@pytest.mark.parametrize("Bn,nH,nKV,T,d", [(2, 16, 4, 256, 128), (1, 4, 2, 96, 64),
                                           (2, 8, 8, 130, 32)])
def test_attention_forward_backward(mi, dev, oracle, Bn, nH, nKV, T, d):
    q, k, v, do = _qkv(oracle, Bn, nH, nKV, T, d, 900 + T)
    Q, K, V, dO = (to_dev(x, dev, True) for x in (q, k, v, do))
    O, P = mi.attention_forward(Q, K, V)
    O_ref, P_ref = oracle.attention_fwd(q, k, v, want_p=True)
    check(host(O), O_ref, TOL_BF16, "O")
    check(host(P), P_ref, TOL_BF16, "P")
    dQ, dK, dV = mi.attention_backward(Q, K, V, dO, P)
    dQ_ref, dK_ref, dV_ref = oracle.attention_bwd(q, k, v, do)
    check(host(dV), dV_ref, TOL_BF16, "dV")
    check(host(dQ), dQ_ref, TOL_BF16, "dQ")
    check(host(dK), dK_ref, TOL_BF16, "dK")


def test_attention_config4_full_size(mi, dev, oracle):
    """Benchmark configuration 4 (B=8, 16 q heads / 4 kv heads, T=1024, d=128): the whole batch
    on the GPU, the oracle on batch elements 0 and 7."""
    Bn, nH, nKV, T, d = 8, 16, 4, 1024, 128
    q, k, v, do = _qkv(oracle, Bn, nH, nKV, T, d, 4000)
    Q, K, V, dO = (to_dev(x, dev, True) for x in (q, k, v, do))
    O, P = mi.attention_forward(Q, K, V)
    dQ, dK, dV = mi.attention_backward(Q, K, V, dO, P)
    Oh, dQh, dKh, dVh = host(O), host(dQ), host(dK), host(dV)
    rows = host(P[:, :, ::97, :]).sum(axis=-1)
    assert np.all(np.abs(rows - 1.0) < 2e-2), "softmax rows must sum to 1"
    for b in (0, 7):
        sl = slice(b, b + 1)
        O_ref = oracle.attention_fwd(q[sl], k[sl], v[sl])
        check(Oh[sl], O_ref, TOL_BF16, f"O[{b}]")
        dQ_ref, dK_ref, dV_ref = oracle.attention_bwd(q[sl], k[sl], v[sl], do[sl])
        check(dQh[sl], dQ_ref, TOL_BF16, f"dQ[{b}]")
        check(dKh[sl], dK_ref, TOL_BF16, f"dK[{b}]")
        check(dVh[sl], dV_ref, TOL_BF16, f"dV[{b}]")


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "f32"])
def test_causal_modes(mi, dev, oracle, bf16):
    """The three causal modes of mi_gemm_batched against dense products with zeros."""
    import torch

    T, d, nb = 200, 64, 3
    tol = TOL_BF16 if bf16 else 1e-4
    low = np.tril(np.ones((T, T), np.float32))
    # OUT_LOWER: S = Q K^T, masked entries take mask_value
    q = inputs(oracle, (nb, T, d), 11, 1.0, bf16)
    kk = inputs(oracle, (nb, T, d), 12, 1.0, bf16)
    S = torch.empty((nb, T, T), dtype=torch.float32, device=dev)
    bt = mi.make_batch(nb, 1, a=(T * d, 0, 1), b=(T * d, 0, 1), c=(T * T, 0, 1),
                       causal=mi.MI_CAUSAL_OUT_LOWER, mask_value=-7.0)
    mi.gemm_batched(to_dev(q, dev, bf16), to_dev(kk, dev, bf16), S, T, T, d, bt, transB=True)
    s = host(S)
    for i in range(nb):
        ref = oracle.gemm(0, 1, T, T, d, q[i], kk[i])
        check(s[i] * low, ref * low, tol, "OUT_LOWER values")
        assert np.all(s[i][low == 0] == -7.0)
    # A_LOWER: C = P V with P lower triangular (k <= m)
    p = inputs(oracle, (nb, T, T), 13, 1.0, bf16) * low
    v = inputs(oracle, (nb, T, d), 14, 1.0, bf16)
    C = torch.empty((nb, T, d), dtype=torch.float32, device=dev)
    bt = mi.make_batch(nb, 1, a=(T * T, 0, 1), b=(T * d, 0, 1), c=(T * d, 0, 1),
                       causal=mi.MI_CAUSAL_A_LOWER)
    mi.gemm_batched(to_dev(p, dev, bf16), to_dev(v, dev, bf16), C, T, d, T, bt)
    c = host(C)
    for i in range(nb):
        check(c[i], oracle.gemm(0, 0, T, d, T, p[i], v[i]), tol, "A_LOWER")
    # A_UPPER with K segments: C = sum_j P_j^T V_j, op(A) = P^T upper triangular
    g = 3
    p = inputs(oracle, (g, T, T), 15, 1.0, bf16) * low
    v = inputs(oracle, (g, T, d), 16, 1.0, bf16)
    C = torch.empty((T, d), dtype=torch.float32, device=dev)
    bt = mi.make_batch(1, 1, k_segments=g, seg_a=T * T, seg_b=T * d, causal=mi.MI_CAUSAL_A_UPPER)
    mi.gemm_batched(to_dev(p, dev, bf16), to_dev(v, dev, bf16), C, T, d, T, bt, transA=True)
    ref = oracle.gemm(1, 0, T, d, T, p, v, nseg=g, segA=T * T, segB=T * d)
    check(host(C), ref, tol, "A_UPPER segments")


# ---- fused flash-attention forward ------------------------------------------------

@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("Bn,nH,nKV,T", [(2, 16, 4, 256), (1, 4, 2, 300), (1, 2, 1, 64),
                                         (1, 4, 4, 520)])
def test_flash_forward(mi, dev, oracle, Bn, nH, nKV, T, d):
    """Fused forward vs the oracle (causal, Attention.cpp:236-280) in both output layouts,
    and the row log-sum-exp vs its closed form; head_dim 128 and 64 (the reference kernel's
    compiled size, flash_attn_fwd.metal:31), both native kernels."""
    import torch

    q, k, v, _ = _qkv(oracle, Bn, nH, nKV, T, d, 1300 + T)
    Q, K, V = (to_dev(x, dev, True) for x in (q, k, v))
    lse = torch.empty((Bn, nH, T), dtype=torch.float32, device=dev)
    O = mi.flash_attn_fwd(Q, K, V, lse=lse)
    O2 = mi.flash_attn_fwd(Q, K, V, layout="bhtd")
    O_ref = oracle.attention_fwd(q, k, v)
    check(host(O), O_ref, TOL_BF16, "O [B,T,nH*d]")
    check(host(O2).transpose(0, 2, 1, 3).reshape(Bn, T, nH * d), O_ref, TOL_BF16, "O [B,nH,T,d]")
    _, lse_ref = dense_attention(q, k, v, True)
    err = np.abs(host(lse) - lse_ref).max()
    assert err < 1e-3, f"lse max abs err {err:.3e}"


@pytest.mark.parametrize("d", [128, 64])
def test_flash_forward_noncausal(mi, dev, oracle, d):
    """causal = 0 attends to every key, including the zero-padded tail block (T % 64 != 0)."""
    Bn, nH, nKV, T = 1, 4, 2, 200
    q, k, v, _ = _qkv(oracle, Bn, nH, nKV, T, d, 1700)
    Q, K, V = (to_dev(x, dev, True) for x in (q, k, v))
    O = mi.flash_attn_fwd(Q, K, V, causal=False, layout="bhtd")
    o_ref, _ = dense_attention(q, k, v, False)
    check(host(O), o_ref, TOL_BF16, "non-causal O")


def test_flash_forward_config4(mi, dev, oracle):
    """Benchmark configuration 4 forward (B=8, 16/4 heads, T=1024, d=128): the fused kernel vs
    the oracle on batch elements 0 and 7 and vs the materialised S/P path on the whole batch."""
    Bn, nH, nKV, T, d = 8, 16, 4, 1024, 128
    q, k, v, _ = _qkv(oracle, Bn, nH, nKV, T, d, 4000)
    Q, K, V = (to_dev(x, dev, True) for x in (q, k, v))
    O = host(mi.flash_attn_fwd(Q, K, V))
    O_mat, _ = mi.attention_forward(Q, K, V)
    check(O, host(O_mat), TOL_BF16, "fused vs materialised")
    for b in (0, 7):
        sl = slice(b, b + 1)
        check(O[sl], oracle.attention_fwd(q[sl], k[sl], v[sl]), TOL_BF16, f"O[{b}]")


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("ws", ["auto", None])
@pytest.mark.parametrize("Bn,nH,nKV,T", [(2, 16, 4, 256), (1, 4, 2, 300), (1, 2, 1, 64),
                                         (1, 4, 4, 520), (1, 2, 1, 130), (2, 4, 1, 200)])
def test_flash_backward(mi, dev, oracle, Bn, nH, nKV, T, ws, d):
    """Fused backward vs the oracle (Attention.cpp:292-348: dV = P^T dO, dS = P (dP - rowsum),
    dQ = scale dS K, dK = scale dS^T Q summed over the query heads of a KV head), in both
    forms: dS^T workspace + batched dQ GEMM ("auto"; T = 300 and 130 are not multiples of 8
    and fall back; 520 and 200 end in a partial query tile) and the dQ kernel (None), at
    head_dim 128 and 64."""
    import torch

    q, k, v, do = _qkv(oracle, Bn, nH, nKV, T, d, 1900 + T)
    Q, K, V, dO = (to_dev(x, dev, True) for x in (q, k, v, do))
    lse = torch.empty((Bn, nH, T), dtype=torch.float32, device=dev)
    O = mi.flash_attn_fwd(Q, K, V, lse=lse)
    print(f"flash backward B={Bn} nH={nH} nKV={nKV} T={T} d={d} workspace={ws}", flush=True)
    dQ, dK, dV = mi.flash_attn_bwd(Q, K, V, O, dO, lse, workspace=ws)
    dQ_ref, dK_ref, dV_ref = oracle.attention_bwd(q, k, v, do)
    check(host(dV), dV_ref, TOL_BF16, "dV")
    check(host(dK), dK_ref, TOL_BF16, "dK")
    check(host(dQ), dQ_ref, TOL_BF16, "dQ")


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("ws", ["auto", None])
def test_flash_backward_noncausal(mi, dev, oracle, ws, d):
    """causal = 0: gradients over every key (T % 64 != 0: a partial last query tile and key
    block) vs the closed form, which is itself pinned to the oracle on the causal case."""
    import torch

    Bn, nH, nKV, T = 1, 4, 2, 200
    q, k, v, do = _qkv(oracle, Bn, nH, nKV, T, d, 2300)
    for ref, got in zip(dense_attention_bwd(q, k, v, do, True), oracle.attention_bwd(q, k, v, do)):
        assert np.abs(ref - got).max() <= 1e-9 * max(1.0, np.abs(got).max())
    Q, K, V, dO = (to_dev(x, dev, True) for x in (q, k, v, do))
    lse = torch.empty((Bn, nH, T), dtype=torch.float32, device=dev)
    O = mi.flash_attn_fwd(Q, K, V, causal=False, lse=lse)
    print(f"flash backward non-causal T={T} workspace={ws}", flush=True)
    dQ, dK, dV = mi.flash_attn_bwd(Q, K, V, O, dO, lse, causal=False, workspace=ws)
    dq_ref, dk_ref, dv_ref = dense_attention_bwd(q, k, v, do, False)
    check(host(dV), dv_ref, TOL_BF16, "dV")
    check(host(dK), dk_ref, TOL_BF16, "dK")
    check(host(dQ), dq_ref, TOL_BF16, "dQ")


@pytest.mark.parametrize("d", [128, 64])
def test_flash_backward_layouts_and_determinism(mi, dev, oracle, d):
    """O/dO in [B,nH,T,d] give the same gradients as [B,T,nH*d], bit for bit, and two
    launches agree bit for bit (no atomics), in the three schedules: dS^T form with the
    balanced dK/dV units (full workspace), dS^T form with one workgroup per key block
    (workspace for dS^T only), and the dQ kernel (no workspace).  The last two share
    the dK/dV kernel and its order of summation: identical dK and dV; the balanced
    units sum partials, equal to them within the bf16 bar."""
    import torch

    Bn, nH, nKV, T = 1, 8, 2, 384
    q, k, v, do = _qkv(oracle, Bn, nH, nKV, T, d, 2100)
    Q, K, V, dO = (to_dev(x, dev, True) for x in (q, k, v, do))
    lse = torch.empty((Bn, nH, T), dtype=torch.float32, device=dev)
    O = mi.flash_attn_fwd(Q, K, V, lse=lse)
    dst_only = torch.empty((Bn * nH * T * T,), dtype=torch.bfloat16, device=dev)
    got = {}
    for name, ws in (("balanced", "auto"), ("per_block", dst_only), ("dq_kernel", None)):
        g1 = mi.flash_attn_bwd(Q, K, V, O, dO, lse, workspace=ws)
        g2 = mi.flash_attn_bwd(Q, K, V, O, dO, lse, workspace=ws)
        O4 = O.view(Bn, T, nH, d).transpose(1, 2).contiguous()
        dO4 = dO.view(Bn, T, nH, d).transpose(1, 2).contiguous()
        g3 = mi.flash_attn_bwd(Q, K, V, O4, dO4, lse, layout="bhtd", workspace=ws)
        for a, b_, c in zip(g1, g2, g3):
            assert torch.equal(a, b_), f"{name}: backward differs between launches"
            assert torch.equal(a, c), f"{name}: backward differs between output layouts"
        got[name] = g1
    assert torch.equal(got["per_block"][1], got["dq_kernel"][1])
    assert torch.equal(got["per_block"][2], got["dq_kernel"][2])
    assert torch.equal(got["per_block"][0], got["balanced"][0])  # same dS^T, same dQ GEMM
    for i, nm in ((1, "dK"), (2, "dV")):
        check(host(got["balanced"][i]), host(got["per_block"][i]).astype(np.float64), TOL_BF16,
              f"balanced {nm}")


def test_flash_backward_config4(mi, dev, oracle):
    """Benchmark configuration 4 backward (B=8, 16/4 heads, T=1024, d=128) vs the oracle on
    batch elements 0 and 7 (the workspace form: key blocks 0-3 of every KV head cut into
    two balanced units each, their partials summed by the reduction kernel)."""
    import torch

    Bn, nH, nKV, T, d = 8, 16, 4, 1024, 128
    q, k, v, do = _qkv(oracle, Bn, nH, nKV, T, d, 4000)
    Q, K, V, dO = (to_dev(x, dev, True) for x in (q, k, v, do))
    lse = torch.empty((Bn, nH, T), dtype=torch.float32, device=dev)
    O = mi.flash_attn_fwd(Q, K, V, lse=lse)
    dQ, dK, dV = (host(t) for t in mi.flash_attn_bwd(Q, K, V, O, dO, lse))
    for b in (0, 7):
        sl = slice(b, b + 1)
        dQ_ref, dK_ref, dV_ref = oracle.attention_bwd(q[sl], k[sl], v[sl], do[sl])
        check(dQ[sl], dQ_ref, TOL_BF16, f"dQ[{b}]")
        check(dK[sl], dK_ref, TOL_BF16, f"dK[{b}]")
        check(dV[sl], dV_ref, TOL_BF16, f"dV[{b}]")


@pytest.mark.parametrize("d", [32, 96])
@pytest.mark.parametrize("layout", ["bthd", "bhtd"])
def test_flash_head_dim_padded(mi, dev, oracle, d, layout):
    """Head dimensions other than 64 and 128 (multiples of 8 below 128) run the next larger
    fused kernels (64 for 32, 128 for 96) on zero-padded rows at the scale 1/sqrt(d)
    (mi_flash_attn_*_scaled): forward, row log-sum-exp and backward vs the oracle, both
    output layouts."""
    import torch

    Bn, nH, nKV, T = 2, 8, 2, 320
    q, k, v, do = _qkv(oracle, Bn, nH, nKV, T, d, 2100 + d)
    Q, K, V, dO = (to_dev(x, dev, True) for x in (q, k, v, do))
    lse = torch.empty((Bn, nH, T), dtype=torch.float32, device=dev)
    print(f"flash head_dim {d} layout {layout}", flush=True)
    O = mi.flash_attn_fwd(Q, K, V, lse=lse, layout=layout)
    O_ref = oracle.attention_fwd(q, k, v)
    got = host(O) if layout == "bthd" else host(O).transpose(0, 2, 1, 3).reshape(Bn, T, nH * d)
    check(got, O_ref, TOL_BF16, f"O d={d}")
    _, lse_ref = dense_attention(q, k, v, True)
    err = np.abs(host(lse) - lse_ref).max()
    assert err < 1e-3, f"lse max abs err {err:.3e}"
    dO_l = dO if layout == "bthd" else dO.reshape(Bn, T, nH, d).permute(0, 2, 1, 3).contiguous()
    dQ, dK, dV = mi.flash_attn_bwd(Q, K, V, O, dO_l, lse, layout=layout)
    dQ_ref, dK_ref, dV_ref = oracle.attention_bwd(q, k, v, do)
    check(host(dV), dV_ref, TOL_BF16, f"dV d={d}")
    check(host(dK), dK_ref, TOL_BF16, f"dK d={d}")
    check(host(dQ), dQ_ref, TOL_BF16, f"dQ d={d}")


def test_flash_config4_head_dim_64(mi, dev, oracle):
    """Configuration 4's batch and heads (B=8, 16 q / 4 kv heads, T=1024) at head_dim 64, the
    reference kernels' compiled size (flash_attn_fwd.metal:31, fused_attn_bwd.metal): the
    native d = 64 forward and backward (dS^T form, balanced schedule) vs the oracle on batch
    elements 0 and 7, and the forward vs the materialised S/P path on the whole batch."""
    import torch

    Bn, nH, nKV, T, d = 8, 16, 4, 1024, 64
    q, k, v, do = _qkv(oracle, Bn, nH, nKV, T, d, 4064)
    Q, K, V, dO = (to_dev(x, dev, True) for x in (q, k, v, do))
    lse = torch.empty((Bn, nH, T), dtype=torch.float32, device=dev)
    print("flash configuration 4 at head_dim 64", flush=True)
    O = mi.flash_attn_fwd(Q, K, V, lse=lse)
    O_mat, _ = mi.attention_forward(Q, K, V)
    Oh = host(O)
    check(Oh, host(O_mat), TOL_BF16, "fused vs materialised (d=64)")
    dQ, dK, dV = (host(t) for t in mi.flash_attn_bwd(Q, K, V, O, dO, lse))
    for b in (0, 7):
        sl = slice(b, b + 1)
        check(Oh[sl], oracle.attention_fwd(q[sl], k[sl], v[sl]), TOL_BF16, f"O[{b}] d=64")
        dQ_ref, dK_ref, dV_ref = oracle.attention_bwd(q[sl], k[sl], v[sl], do[sl])
        check(dQ[sl], dQ_ref, TOL_BF16, f"dQ[{b}] d=64")
        check(dK[sl], dK_ref, TOL_BF16, f"dK[{b}] d=64")
        check(dV[sl], dV_ref, TOL_BF16, f"dV[{b}] d=64")


def test_flash_backward_graph_replays(mi, dev):
    """The dS^T-form backward (D, dK/dV with the balanced schedule, the partial sums and
    the dQ GEMM) captured in a HIP graph: every replay, with eager launches and
    synchronisations between replays, gives the eager result bit for bit."""
    import torch

    Bn, nH, nKV, T, d = 2, 16, 4, 1024, 128
    g = torch.Generator(device=dev)
    g.manual_seed(31)
    Q = torch.randn((Bn, nH, T, d), generator=g, device=dev).to(torch.bfloat16)
    K = torch.randn((Bn, nKV, T, d), generator=g, device=dev).to(torch.bfloat16)
    V = torch.randn((Bn, nKV, T, d), generator=g, device=dev).to(torch.bfloat16)
    dO = (torch.randn((Bn, T, nH * d), generator=g, device=dev) * 1e-2).to(torch.bfloat16)
    lse = torch.empty((Bn, nH, T), dtype=torch.float32, device=dev)
    O = mi.flash_attn_fwd(Q, K, V, lse=lse)
    ws = torch.empty((mi.load_library().mi_flash_attn_bwd_workspace_size(Bn, nH, T) // 2,),
                     dtype=torch.bfloat16, device=dev)
    print("flash backward graph: eager reference", flush=True)
    ref = [t.clone() for t in mi.flash_attn_bwd(Q, K, V, O, dO, lse, workspace=ws)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mi.flash_attn_bwd(Q, K, V, O, dO, lse, sync=False, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print("flash backward graph: capture", flush=True)
    with torch.cuda.graph(graph):
        out = mi.flash_attn_bwd(Q, K, V, O, dO, lse, sync=False, workspace=ws)
    for i in range(3):
        print(f"flash backward graph: replay {i}", flush=True)
        for t in out:
            t.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(out, ref):
            assert torch.equal(got, want), i
        eager = mi.flash_attn_bwd(Q, K, V, O, dO, lse, workspace=ws)
        for got, want in zip(eager, ref):
            assert torch.equal(got, want), i
