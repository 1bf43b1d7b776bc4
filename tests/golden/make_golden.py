"""Writes tests/golden/*.npz: small seeded GEMM / attention cases with float64
expected outputs from the CPU oracle (oracle/mi_oracle.c), plus the reference's
own known answers (reference_kats.json, copied as data from
cpp/tests/test_math_ops.cpp:167-189).

Run from the repository root:  python tests/golden/make_golden.py
The fixtures are committed; tests/test_golden.py checks the oracle still
reproduces them bit-for-bit and tests/test_golden_gpu.py checks the HIP path
against the stored expectations.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle  # noqa: E402


def _bf(x):
    return oracle.round_bf16(x)


def gemm_cases():
    cases = {}
    M, N, K = 17, 33, 65
    for tA in (0, 1):
        for tB in (0, 1):
            a = _bf(oracle.normal((M, K), 1 + 2 * tA + tB))
            b = _bf(oracle.normal((K, N), 11 + 2 * tA + tB, 0.0, 0.05))
            A = np.ascontiguousarray(a.T) if tA else a
            B = np.ascontiguousarray(b.T) if tB else b
            cases[f"bf16_t{tA}{tB}"] = dict(
                tA=tA, tB=tB, M=M, N=N, K=K, bf16=1, A=A, B=B,
                expected=oracle.gemm(tA, tB, M, N, K, A, B))
    M, N, K = 24, 40, 48
    a = oracle.normal((M, K), 21)
    w = oracle.normal((N, K), 22, 0.0, 0.02)
    bias = oracle.normal((N,), 23, 0.0, 0.02)
    cases["f32_linear_bias"] = dict(tA=0, tB=1, M=M, N=N, K=K, bf16=0, A=a, B=w, bias=bias,
                                    expected=oracle.gemm(0, 1, M, N, K, a, w, bias=bias))
    M, N, K = 32, 48, 100
    x = _bf(oracle.normal((K, M), 31))
    dy = _bf(oracle.normal((K, N), 32, 0.0, 1e-2))
    c0 = oracle.normal((M, N), 33, 0.0, 1e-3)
    cases["bf16_dw_accumulate"] = dict(tA=1, tB=0, M=M, N=N, K=K, bf16=1, A=x, B=dy, C0=c0,
                                       beta=1.0,
                                       expected=oracle.gemm(1, 0, M, N, K, x, dy, beta=1.0, C0=c0))
    M, N, K = 20, 36, 44
    a = _bf(oracle.normal((M, K), 41))
    bg = _bf(oracle.normal((K, N), 42, 0.0, 0.2))
    bu = _bf(oracle.normal((K, N), 43, 0.0, 0.2))
    cases["bf16_dual_silu"] = dict(tA=0, tB=0, M=M, N=N, K=K, bf16=1, A=a, B=bg, B2=bu,
                                   expected=oracle.gemm(0, 0, M, N, K, a, bg, B2=bu, mode=1))
    g = _bf(oracle.normal((M, K), 44))
    u = _bf(oracle.normal((M, K), 45))
    b = _bf(oracle.normal((K, N), 46, 0.0, 0.1))
    cases["bf16_prologue_silu"] = dict(tA=0, tB=0, M=M, N=N, K=K, bf16=1, A=g, A2=u, B=b,
                                       expected=oracle.gemm(0, 0, M, N, K, g, b, A2=u, mode=2))
    return cases


def attention_case():
    Bn, nH, nKV, T, d = 1, 4, 2, 16, 16
    q = _bf(oracle.normal((Bn, nH, T, d), 51))
    k = _bf(oracle.normal((Bn, nKV, T, d), 52))
    v = _bf(oracle.normal((Bn, nKV, T, d), 53))
    do = _bf(oracle.normal((Bn, T, nH * d), 54, 0.0, 1e-2))
    O = oracle.attention_fwd(q, k, v)
    dQ, dK, dV = oracle.attention_bwd(q, k, v, do)
    return dict(Q=q, K=k, V=v, dO=do, O=O, dQ=dQ, dK=dK, dV=dV)


def main():
    flat = {}
    for name, c in gemm_cases().items():
        for key, val in c.items():
            flat[f"{name}__{key}"] = np.asarray(val)
    np.savez_compressed(os.path.join(HERE, "gemm_cases.npz"), **flat)
    np.savez_compressed(os.path.join(HERE, "attention_case.npz"), **attention_case())
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
