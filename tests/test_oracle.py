"""Pins the CPU oracle (oracle/mi_oracle.c) before it is trusted as the checker.

Each check compares the oracle with something it was not derived from: the
reference's own known answers (TC-12/TC-13, test_math_ops.cpp:167-189), numpy's
float64/int64 matmul (a library routine), scipy's logistic function, dense
matrix formulations of attention, finite differences of the oracle's own forward
pass (test_backward.cpp:104-151 uses the same central-difference scheme), torch's
bf16 rounding, and exact small-integer arithmetic. Each is chosen so that a
dropped term, a wrong sign or index, or a transposed operand fails it.
"""
import numpy as np
import pytest
from scipy.special import expit


def _rng(seed):
    return np.random.default_rng(seed)


def _store(op, trans, ld_pad=0):
    """Lay out the logical operand op [R, C] for the given transpose flag with padding."""
    rows, cols = (op.shape[1], op.shape[0]) if trans else op.shape
    buf = np.zeros((rows, cols + ld_pad), dtype=np.float32)
    buf[:, :cols] = op.T if trans else op
    return buf, cols + ld_pad


def test_kat_tc12(oracle):
    A = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    B = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    C = oracle.gemm(0, 0, 2, 2, 3, A, B)
    assert C.tolist() == [[58.0, 64.0], [139.0, 154.0]]


def test_kat_tc13_batched(oracle):
    A = np.array([1, 2, 3, 4, 5, 6, 1, 1, 1, 2, 2, 2], np.float32).reshape(2, 2, 3)
    B = np.array([7, 8, 9, 10, 11, 12, 1, 2, 3, 4, 5, 6], np.float32).reshape(2, 3, 2)
    C = np.stack([oracle.gemm(0, 0, 2, 2, 3, A[b], B[b]) for b in range(2)])
    assert C[0, 0, 0] == 58.0 and C[1, 1, 1] == 24.0


@pytest.mark.parametrize("tA,tB", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_transposes_vs_numpy(oracle, tA, tB):
    rng = _rng(10 + 2 * tA + tB)
    M, N, K = 17, 33, 65
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    A, lda = _store(a, tA, ld_pad=3)
    B, ldb = _store(b, tB, ld_pad=5)
    C = oracle.gemm(tA, tB, M, N, K, A, B, lda=lda, ldb=ldb, alpha=0.75)
    ref = 0.75 * (a.astype(np.float64) @ b.astype(np.float64))
    assert np.max(np.abs(C - ref)) <= 1e-12 * np.max(np.abs(ref))
    # a transposed operand would not match
    assert np.max(np.abs(C - 0.75 * (a.astype(np.float64) @ b.astype(np.float64)[:, ::-1]))) > 1e-3


def test_integer_exact(oracle):
    rng = _rng(3)
    M, N, K = 40, 24, 56
    a = rng.integers(-8, 9, (M, K))
    b = rng.integers(-8, 9, (K, N))
    C = oracle.gemm(0, 0, M, N, K, a.astype(np.float32), b.astype(np.float32))
    assert np.array_equal(C, (a @ b).astype(np.float64))


def test_linearity_tc20(oracle):
    """(A1 + 2 A2) B = A1 B + 2 A2 B and A (B1 + B2) = A B1 + A B2
    (TC-20, test_transformer.cpp:450-482), in the NT layout of a projection."""
    rng = _rng(21)
    M, N, K = 23, 19, 37
    a1, a2 = (rng.standard_normal((M, K)) for _ in range(2))
    b1, b2 = (rng.standard_normal((N, K)) for _ in range(2))
    g = lambda a, b: oracle.gemm(0, 1, M, N, K, a.astype(np.float32), b.astype(np.float32))
    f32 = lambda x: x.astype(np.float32).astype(np.float64)
    lhs = g(f32(a1) + 2 * f32(a2), b1)
    assert np.allclose(lhs, g(a1, b1) + 2 * g(a2, b1), rtol=1e-6, atol=1e-6)
    assert np.allclose(g(a1, f32(b1) + f32(b2)), g(a1, b1) + g(a1, b2), rtol=1e-6, atol=1e-6)


def test_transpose_identity(oracle):
    """(A B)^T = B^T A^T: the TN product of stored operands equals the transpose of
    the NT product with the operands swapped."""
    rng = _rng(22)
    M, N, K = 14, 31, 26
    x = rng.standard_normal((K, M)).astype(np.float32)   # activations [tokens, in]
    dy = rng.standard_normal((K, N)).astype(np.float32)  # gradient [tokens, out]
    dw = oracle.gemm(1, 0, M, N, K, x, dy)                # x^T dy
    dwt = oracle.gemm(1, 0, N, M, K, dy, x)               # dy^T x
    assert np.allclose(dw, dwt.T, rtol=1e-12, atol=1e-12)
    assert not np.allclose(dw[:, :M], dwt[:M, :], atol=1e-3)


def test_accumulate_tc28(oracle):
    """Two backward passes accumulate into one weight gradient with beta = 1
    (TC-28, test_transformer.cpp:615-636; Transformer.cpp:236,288-289)."""
    rng = _rng(23)
    M, N, K = 16, 12, 40
    x1, x2 = (rng.standard_normal((K, M)).astype(np.float32) for _ in range(2))
    d1, d2 = (rng.standard_normal((K, N)).astype(np.float32) for _ in range(2))
    g1 = oracle.gemm(1, 0, M, N, K, x1, d1)
    acc = oracle.gemm(1, 0, M, N, K, x2, d2, beta=1.0, C0=g1.astype(np.float32))
    ref = x1.T.astype(np.float64) @ d1 + x2.T.astype(np.float64) @ d2
    assert np.allclose(acc, ref, rtol=1e-6, atol=1e-6)
    # overwrite semantics (beta = 0) would drop the first pass
    assert np.max(np.abs(oracle.gemm(1, 0, M, N, K, x2, d2) - ref)) > 1e-2


def test_epilogue_bias_beta_residual(oracle):
    rng = _rng(4)
    M, N, K = 12, 20, 9
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((N, K)).astype(np.float32)  # nn.Linear layout: Y = X W^T + b
    bias = rng.standard_normal(N).astype(np.float32)
    c0 = rng.standard_normal((M, N)).astype(np.float32)
    r = rng.standard_normal((M, N)).astype(np.float32)
    C = oracle.gemm(0, 1, M, N, K, a, b, alpha=2.0, beta=0.5, C0=c0, bias=bias, R=r)
    ref = 2.0 * (a.astype(np.float64) @ b.T.astype(np.float64)) + bias[None, :] + 0.5 * c0 + r
    assert np.allclose(C, ref, rtol=1e-12, atol=1e-12)


def test_dual_silu_gate(oracle):
    rng = _rng(5)
    M, N, K = 10, 14, 22
    a = rng.standard_normal((M, K)).astype(np.float32)
    bg = rng.standard_normal((K, N)).astype(np.float32)
    bu = rng.standard_normal((K, N)).astype(np.float32)
    C = oracle.gemm(0, 0, M, N, K, a, bg, B2=bu, mode=1)
    g = a.astype(np.float64) @ bg.astype(np.float64)
    u = a.astype(np.float64) @ bu.astype(np.float64)
    assert np.allclose(C, g * expit(g) * u, rtol=1e-12, atol=1e-12)


def test_prologue_silu_gate(oracle):
    rng = _rng(6)
    M, N, K = 9, 11, 30
    g = rng.standard_normal((M, K)).astype(np.float32) * 3
    u = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    C = oracle.gemm(0, 0, M, N, K, g, b, A2=u, mode=2)
    act = g.astype(np.float64) * expit(g.astype(np.float64)) * u
    assert np.allclose(C, act @ b.astype(np.float64), rtol=1e-12, atol=1e-12)


def test_k_segments_sum(oracle):
    """K segments at arbitrary strides equal the sum of the per-segment products."""
    rng = _rng(7)
    M, N, K, S = 6, 5, 8, 3
    a = rng.standard_normal((S, M, 20)).astype(np.float32)  # segment j: a[j, :, :K], lda=20
    b = rng.standard_normal((S, K, 7)).astype(np.float32)   # segment j: b[j, :, :N], ldb=7
    C = oracle.gemm(0, 0, M, N, K, a, b, lda=20, ldb=7, nseg=S, segA=M * 20, segB=K * 7)
    ref = sum(a[j, :, :K].astype(np.float64) @ b[j, :, :N].astype(np.float64) for j in range(S))
    assert np.allclose(C, ref, rtol=1e-12, atol=1e-12)


def test_sampled_rows(oracle):
    rng = _rng(8)
    M, N, K = 30, 7, 9
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    full = oracle.gemm(0, 0, M, N, K, a, b)
    rows = np.array([29, 0, 13], dtype=np.int64)
    part = oracle.gemm(0, 0, M, N, K, a, b, rows=rows)
    assert np.array_equal(part, full[rows])


def _dense_attention(Q, K, V):
    """softmax(Q K^T / sqrt(d) + causal mask) V with the GQA head map, float64."""
    Bn, nH, T, d = Q.shape
    g = nH // K.shape[1]
    Kx = np.repeat(K.astype(np.float64), g, axis=1)
    Vx = np.repeat(V.astype(np.float64), g, axis=1)
    S = np.einsum("bhqd,bhkd->bhqk", Q.astype(np.float64), Kx) / np.sqrt(d)
    S = np.where(np.tril(np.ones((T, T), bool)), S, -np.inf)
    P = np.exp(S - S.max(-1, keepdims=True))
    P /= P.sum(-1, keepdims=True)
    O = np.einsum("bhqk,bhkd->bhqd", P, Vx)
    return O.transpose(0, 2, 1, 3).reshape(Bn, T, nH * d), P


def test_attention_fwd_vs_dense(oracle):
    rng = _rng(9)
    Bn, nH, nKV, T, d = 2, 4, 2, 12, 8
    Q = rng.standard_normal((Bn, nH, T, d)).astype(np.float32)
    K = rng.standard_normal((Bn, nKV, T, d)).astype(np.float32)
    V = rng.standard_normal((Bn, nKV, T, d)).astype(np.float32)
    O, P = oracle.attention_fwd(Q, K, V, want_p=True)
    Od, Pd = _dense_attention(Q, K, V)
    assert np.allclose(O, Od, rtol=1e-12, atol=1e-12)
    assert np.allclose(P, Pd, rtol=1e-12, atol=1e-12)
    # causal: future keys do not influence earlier rows (test_attention.cpp:99-114)
    V2 = V.copy()
    V2[:, :, -1, :] += 100.0
    O2 = oracle.attention_fwd(Q, K, V2)
    assert np.array_equal(O2[:, :-1], O[:, :-1])


def test_attention_bwd_finite_difference(oracle):
    """Gradients of L = sum(O * G) against central differences of the forward."""
    rng = _rng(10)
    Bn, nH, nKV, T, d = 1, 4, 2, 6, 4
    Q = rng.standard_normal((Bn, nH, T, d)).astype(np.float32)
    K = rng.standard_normal((Bn, nKV, T, d)).astype(np.float32)
    V = rng.standard_normal((Bn, nKV, T, d)).astype(np.float32)
    G = rng.standard_normal((Bn, T, nH * d)).astype(np.float32)
    dQ, dK, dV = oracle.attention_bwd(Q, K, V, G)
    eps = 1e-3

    def loss(q, k, v):
        return float(np.sum(oracle.attention_fwd(q, k, v) * G))

    for name, X, dX in (("Q", Q, dQ), ("K", K, dK), ("V", V, dV)):
        for idx in [(0, 0, 0, 0), (0, 1, 3, 2), (0, X.shape[1] - 1, T - 1, d - 1), (0, 0, 2, 1)]:
            Xp, Xm = X.copy(), X.copy()
            Xp[idx] += eps
            Xm[idx] -= eps
            args_p = {"Q": Q, "K": K, "V": V}
            args_m = {"Q": Q, "K": K, "V": V}
            args_p[name], args_m[name] = Xp, Xm
            # the float32 perturbation actually applied
            h = float(np.float64(Xp[idx]) - np.float64(Xm[idx]))
            fd = (loss(args_p["Q"], args_p["K"], args_p["V"]) -
                  loss(args_m["Q"], args_m["K"], args_m["V"])) / h
            assert abs(fd - dX[idx]) <= 1e-4 * max(1.0, abs(fd)), (name, idx, fd, dX[idx])


def test_bf16_conversions(oracle):
    import torch

    x = np.concatenate([_rng(11).standard_normal(10000).astype(np.float32) * 100,
                        np.array([0.0, -0.0, 1.0, 3.0000002, 65504.0, 1e-40, -2.5e-38,
                                  np.inf, -np.inf], np.float32)])
    trunc = oracle.to_bf16(x, rne=False)
    assert np.array_equal(trunc, (x.view(np.uint32) >> 16).astype(np.uint16))  # Tensor.hpp:16-20
    rne = oracle.to_bf16(x, rne=True)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(rne, ref)
    back = oracle.from_bf16(rne)
    assert np.array_equal(back, torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_normal_generator(oracle):
    a = oracle.normal((1 << 20,), 123, 0.5, 2.0)
    b = oracle.normal((1 << 20,), 123, 0.5, 2.0)
    assert np.array_equal(a, b)
    assert abs(a.mean() - 0.5) < 0.01 and abs(a.std() - 2.0) < 0.01
    # prefix property: a shorter draw is a prefix of a longer one
    assert np.array_equal(oracle.normal((1001,), 123, 0.5, 2.0), a[:1001])
    assert not np.array_equal(oracle.normal((1000,), 124, 0.5, 2.0), a[:1000])


@pytest.mark.parametrize("tA,tB", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_baseline(oracle, tA, tB):
    rng = _rng(12 + tA + 2 * tB)
    M, N, K = 70, 300, 260
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    A = np.ascontiguousarray(a.T) if tA else a
    B = np.ascontiguousarray(b.T) if tB else b
    C = oracle.sgemm_omp(tA, tB, M, N, K, A, B)
    assert oracle.max_rel_err(C, a.astype(np.float64) @ b.astype(np.float64)) < 1e-5


def test_error_metrics(oracle):
    assert oracle.l2_rel_err([3.0, 4.5], [3.0, 4.0]) == pytest.approx(0.1)
    assert oracle.max_rel_err([1.0, 2.5], [1.0, 2.0]) == pytest.approx(0.25)
