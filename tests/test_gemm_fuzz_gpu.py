"""Seeded sweep of mi_gemm over tile-boundary shapes, layouts, dtypes, leading-dimension
padding and epilogues (alpha, beta*C, bias, residual, split-K through a workspace), each
case against the float64 oracle at the fp32 / bf16 bar. The shapes straddle the 32-row
MFMA blocks and the 64/128/192/256 tiles, so edge tiles, K tails, the direct and the
general epilogue, the direct-to-LDS and the register-staged kernels all take part."""
import numpy as np
import pytest

from gpu_cases import TOL_BF16, TOL_F32
from test_gemm_gpu import _run
from gpu_cases import check

pytestmark = pytest.mark.gpu

SIZES = [1, 7, 31, 32, 33, 63, 64, 65, 100, 127, 128, 129, 191, 192, 193, 255, 256, 257, 320, 384,
         511, 520]


def _cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        c = dict(M=int(rng.choice(SIZES)), N=int(rng.choice(SIZES)), K=int(rng.choice(SIZES)),
                 tA=int(rng.integers(2)), tB=int(rng.integers(2)), bf16=bool(rng.integers(2)),
                 out_bf16=bool(rng.integers(2)),
                 pad=tuple(int(x) for x in rng.choice([0, 0, 8, 3], size=3)),
                 alpha=float(rng.choice([1.0, 0.5])), beta=float(rng.choice([0.0, 0.0, 1.0, -0.5])),
                 bias=bool(rng.integers(2)), residual=bool(rng.random() < 0.3),
                 ws=bool(rng.integers(2)))
        out.append(c)
    return out


@pytest.mark.parametrize("part", range(4))
def test_gemm_sweep(mi, dev, oracle, part):
    import torch

    ws = torch.empty(4 << 20, dtype=torch.float32, device=dev)
    for i, c in enumerate(_cases(48, 4000 + part)):
        tol = TOL_BF16 if (c["bf16"] or c["out_bf16"]) else TOL_F32
        got, ref = _run(mi, dev, oracle, c["M"], c["N"], c["K"], c["tA"], c["tB"], c["bf16"],
                        seed=7000 + 100 * part + i, out_bf16=c["out_bf16"], alpha=c["alpha"],
                        beta=c["beta"], bias=c["bias"], residual=c["residual"], pad=c["pad"],
                        ws=ws if c["ws"] else None)
        check(got, ref, tol, f"case {part}.{i} {c}")


@pytest.mark.parametrize("part", range(2))
def test_dual_and_prologue_sweep(mi, dev, oracle, part):
    """The dual-B SiLU-gate product (gemm_ffn) and the SiLU-gate A prologue
    (fused_swiglu_gemm) over random shapes, layouts (the prologue needs A
    K-contiguous) and dtypes, with and without a workspace (the bf16 prologue's
    two-pass form), against the oracle."""
    import torch

    rng = np.random.default_rng(5000 + part)
    ws = torch.empty(4 << 20, dtype=torch.float32, device=dev)
    for i in range(16):
        M, N, K = (int(rng.choice(SIZES)) for _ in range(3))
        bf16 = bool(rng.integers(2))
        prologue = bool(rng.integers(2))
        tA = 0 if prologue else int(rng.integers(2))
        tB = int(rng.integers(2))
        beta = float(rng.choice([0.0, 1.0]))
        use_ws = bool(rng.integers(2))
        got, ref = _run(mi, dev, oracle, M, N, K, tA, tB, bf16, seed=9000 + 100 * part + i,
                        dual=not prologue, prologue=prologue, beta=beta, ws=ws if use_ws else None)
        check(got, ref, TOL_BF16 if bf16 else TOL_F32,
              f"{'prologue' if prologue else 'dual'} {M}x{N}x{K} tA={tA} tB={tB} bf16={bf16} beta={beta} ws={use_ws}")


@pytest.mark.parametrize("part", range(2))
def test_batched_sweep(mi, dev, oracle, part):
    """mi_gemm_batched over random batch x heads problems with a head map (A, B or C
    shared by groups of heads), K segments, layouts and dtypes, against the oracle per
    problem."""
    import torch

    from gpu_cases import host, inputs, layout, to_dev

    rng = np.random.default_rng(6000 + part)
    for i in range(12):
        nb, heads = int(rng.integers(1, 3)), int(rng.choice([1, 2, 4]))
        gb = int(rng.choice([g for g in (1, 2, 4) if heads % g == 0]))
        M, N, K = (int(rng.choice(SIZES[3:17])) for _ in range(3))
        nseg = int(rng.choice([1, 1, 2]))
        tA, tB = int(rng.integers(2)), int(rng.integers(2))
        bf16 = bool(rng.integers(2))
        tol = TOL_BF16 if bf16 else TOL_F32
        seed = 11000 + 100 * part + 10 * i
        a = inputs(oracle, (nb, heads, nseg, M, K), seed, 1.0, bf16)
        b = inputs(oracle, (nb, heads // gb, nseg, K, N), seed + 1, 0.05, bf16)
        A = np.stack([[[layout(a[x, h, s], tA) for s in range(nseg)] for h in range(heads)]
                      for x in range(nb)])
        B = np.stack([[[layout(b[x, h, s], tB) for s in range(nseg)] for h in range(heads // gb)]
                      for x in range(nb)])
        C = torch.zeros((nb, heads, M, N), dtype=torch.float32, device=dev)
        bt = mi.make_batch(nb * heads, heads, a=(heads * nseg * M * K, nseg * M * K, 1),
                           b=((heads // gb) * nseg * K * N, nseg * K * N, gb),
                           c=(heads * M * N, M * N, 1), k_segments=nseg, seg_a=M * K, seg_b=K * N)
        mi.gemm_batched(to_dev(A, dev, bf16), to_dev(B, dev, bf16), C, M, N, K, bt, transA=tA,
                        transB=tB)
        got = host(C)
        for x in range(nb):
            for h in range(heads):
                ref = sum(oracle.gemm(0, 0, M, N, K, a[x, h, s], b[x, h // gb, s]) for s in range(nseg))
                check(got[x, h], ref, tol, f"batched case {part}.{i} problem ({x},{h}) "
                      f"{M}x{N}x{K} tA={tA} tB={tB} bf16={bf16} nseg={nseg} group={gb}")
