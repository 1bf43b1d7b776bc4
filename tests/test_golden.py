"""The oracle reproduces the committed fixtures (tests/golden/) exactly, and the
reference's own known answers (reference_kats.json, test_math_ops.cpp:167-189)."""
import json
import os

import numpy as np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_gemm_cases():
    z = np.load(os.path.join(HERE, "gemm_cases.npz"))
    cases = {}
    for key in z.files:
        name, field = key.split("__")
        cases.setdefault(name, {})[field] = z[key]
    return cases


def _oracle_for(oracle, c):
    mode = 1 if "B2" in c else (2 if "A2" in c else 0)
    return oracle.gemm(int(c["tA"]), int(c["tB"]), int(c["M"]), int(c["N"]), int(c["K"]), c["A"],
                       c["B"], bias=c.get("bias"), beta=float(c.get("beta", 0.0)), C0=c.get("C0"),
                       B2=c.get("B2"), A2=c.get("A2"), mode=mode)


def test_gemm_fixtures(oracle):
    cases = load_gemm_cases()
    assert len(cases) >= 8
    for name, c in cases.items():
        assert np.array_equal(_oracle_for(oracle, c), c["expected"]), name


def test_attention_fixture(oracle):
    z = np.load(os.path.join(HERE, "attention_case.npz"))
    assert np.array_equal(oracle.attention_fwd(z["Q"], z["K"], z["V"]), z["O"])
    dQ, dK, dV = oracle.attention_bwd(z["Q"], z["K"], z["V"], z["dO"])
    assert np.array_equal(dQ, z["dQ"]) and np.array_equal(dK, z["dK"])
    assert np.array_equal(dV, z["dV"])


def test_reference_kats(oracle):
    k = json.load(open(os.path.join(HERE, "reference_kats.json")))
    A = np.array(k["tc12"]["A"], np.float32)
    B = np.array(k["tc12"]["B"], np.float32)
    assert oracle.gemm(0, 0, 2, 2, 3, A, B).tolist() == k["tc12"]["expected"]
    A3 = np.array(k["tc13"]["A"], np.float32)
    B3 = np.array(k["tc13"]["B"], np.float32)
    assert oracle.gemm(0, 0, 2, 2, 3, A3[0], B3[0])[0, 0] == k["tc13"]["expected_000"]
    assert oracle.gemm(0, 0, 2, 2, 3, A3[1], B3[1])[1, 1] == k["tc13"]["expected_111"]
