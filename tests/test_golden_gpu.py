"""The HIP path against the committed golden fixtures (tests/golden/), through the C ABI."""
import os

import numpy as np
import pytest

from gpu_cases import TOL_BF16, TOL_F32, check, host, to_dev
from test_golden import HERE, load_gemm_cases

pytestmark = pytest.mark.gpu


def test_gemm_fixtures_gpu(mi, dev):
    import torch

    for name, c in load_gemm_cases().items():
        bf = bool(c["bf16"])
        M, N, K = int(c["M"]), int(c["N"]), int(c["K"])
        kw = {}
        for key in ("bias", "B2", "A2"):
            if key in c:
                kw[key] = to_dev(c[key], dev, bf)
        beta = float(c["beta"]) if "beta" in c else 0.0
        if "C0" in c:
            C = torch.from_numpy(c["C0"].astype(np.float32)).to(dev)
        else:
            C = torch.zeros((M, N), dtype=torch.float32, device=dev)
        mi.gemm(to_dev(c["A"], dev, bf), to_dev(c["B"], dev, bf), C, M, N, K,
                transA=int(c["tA"]), transB=int(c["tB"]), beta=beta, **kw)
        check(host(C), c["expected"], TOL_BF16 if bf else TOL_F32, name)


def test_attention_fixture_gpu(mi, dev):
    z = np.load(os.path.join(HERE, "attention_case.npz"))
    Q, K, V, dO = (to_dev(z[k], dev, True) for k in ("Q", "K", "V", "dO"))
    O, P = mi.attention_forward(Q, K, V)
    check(host(O), z["O"], TOL_BF16, "O")
    dQ, dK, dV = mi.attention_backward(Q, K, V, dO, P)
    check(host(dQ), z["dQ"], TOL_BF16, "dQ")
    check(host(dK), z["dK"], TOL_BF16, "dK")
    check(host(dV), z["dV"], TOL_BF16, "dV")
