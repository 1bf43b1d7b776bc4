"""Seeded sweep of the fused attention (Attention.cpp:236-280 forward, 292-348 backward;
the Metal kernels' entry points MetalBridge.hpp:49-57) over random shapes: batch, KV heads,
query heads per KV head, sequence lengths on and off the 64-row block and 8-query run
boundaries, head_dim 64 and 128 (native) and 32 and 96 (padded), causal or not, both O
layouts, and the backward with and without the dS^T workspace.  Every case is checked
against the float64 closed forms (pinned to the oracle on the causal case in
test_attention_gpu.py) at the bf16 bar.
"""
import numpy as np
import pytest

from gpu_cases import TOL_BF16, check, dense_attention, dense_attention_bwd, host, inputs, to_dev

pytestmark = pytest.mark.gpu

SEQ = [1, 7, 8, 63, 64, 65, 127, 128, 129, 136, 200, 256, 300, 384]
HEAD_DIMS = [64, 128, 128, 64, 32, 96]


def _cases(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        Bn = int(rng.integers(1, 3))
        nKV = int(rng.integers(1, 4))
        g = int(rng.choice([1, 2, 4]))
        T = int(rng.choice(SEQ))
        d = int(rng.choice(HEAD_DIMS))
        causal = bool(rng.integers(0, 2))
        layout = "bthd" if rng.integers(0, 2) else "bhtd"
        ws = "auto" if rng.integers(0, 2) else None
        out.append((Bn, nKV * g, nKV, T, d, causal, layout, ws, int(rng.integers(1 << 20))))
    return out


@pytest.mark.parametrize("part", range(3))
def test_flash_sweep(mi, dev, oracle, part):
    import torch

    for Bn, nH, nKV, T, d, causal, lay, ws, seed in _cases(7100 + part, 10):
        print(f"flash sweep B={Bn} nH={nH} nKV={nKV} T={T} d={d} causal={causal} "
              f"layout={lay} workspace={ws} seed={seed}", flush=True)
        q = inputs(oracle, (Bn, nH, T, d), seed)
        k = inputs(oracle, (Bn, nKV, T, d), seed + 1)
        v = inputs(oracle, (Bn, nKV, T, d), seed + 2)
        do = inputs(oracle, (Bn, T, nH * d), seed + 3, 1e-2)
        Q, K, V = (to_dev(x, dev, True) for x in (q, k, v))
        lse = torch.empty((Bn, nH, T), dtype=torch.float32, device=dev)
        O = mi.flash_attn_fwd(Q, K, V, lse=lse, causal=causal, layout=lay)
        o_ref, lse_ref = dense_attention(q, k, v, causal)
        o = host(O)
        if lay == "bthd":
            o = o.reshape(Bn, T, nH, d).transpose(0, 2, 1, 3)
        check(o, o_ref, TOL_BF16, "O")
        err = np.abs(host(lse) - lse_ref).max()
        assert err < 1e-3, f"lse max abs err {err:.3e}"
        dO = to_dev(do, dev, True)
        if lay == "bhtd":
            dO = dO.view(Bn, T, nH, d).transpose(1, 2).contiguous()
        dQ, dK, dV = mi.flash_attn_bwd(Q, K, V, O, dO, lse, causal=causal, layout=lay, workspace=ws)
        dq_ref, dk_ref, dv_ref = dense_attention_bwd(q, k, v, do, causal)
        check(host(dV), dv_ref, TOL_BF16, "dV")
        check(host(dK), dk_ref, TOL_BF16, "dK")
        check(host(dQ), dq_ref, TOL_BF16, "dQ")
