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
