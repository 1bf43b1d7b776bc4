"""Seeded sweep of the LM head + cross-entropy over vocabulary chunks (mi_lm_head_xent; the
reference's logits = final_h.matmul(output_projection_), Transformer.cpp:193-194, its
CrossEntropyLoss, Loss.cpp:43-195, and the output projection's backward, Transformer.cpp:
600-616) over random problems: row counts, hidden sizes, vocabularies and chunk sizes on
and off whole 16-byte vectors and 64-column slices, both weight layouts, dX and dW in bf16
or fp32 or skipped, dW overwritten or accumulated.  Every case is checked against the
oracle as in test_lm_head_gpu.py: bf16 logits, the oracle's cross-entropy, the bf16
gradient, then the two products in float64 (row losses within 2e-3 * max(1, |ref|), dX and
dW within 1e-2 of their largest magnitude).
"""
import numpy as np
import pytest

from gpu_cases import TOL_BF16, check, host, inputs, to_dev

pytestmark = pytest.mark.gpu


def _cases(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        rows = int(rng.choice([1, 7, 64, 100, 257]))
        hidden = int(8 * rng.integers(2, 49))
        vocab = int(rng.choice([int(rng.integers(2, 5000)), 8 * int(rng.integers(1, 700))]))
        chunk = int(rng.choice([0, 64 * int(rng.integers(1, 33)), int(rng.integers(1, 3000))]))
        layout = int(rng.integers(0, 2))
        dxt = [None, "bf16", "f32"][int(rng.integers(0, 3))]
        dwt = [None, "bf16", "f32"][int(rng.integers(0, 3))]
        beta = float(rng.choice([0.0, 1.0]))
        out.append((rows, hidden, vocab, chunk, layout, dxt, dwt, beta, int(rng.integers(1 << 20))))
    return out


@pytest.mark.parametrize("part", range(2))
def test_lm_head_xent_sweep(mi, dev, oracle, part):
    import torch

    tdt = {"bf16": torch.bfloat16, "f32": torch.float32}
    for rows, hidden, vocab, chunk, layout, dxt, dwt, beta, seed in _cases(8300 + part, 12):
        print(f"lm_head_xent sweep rows={rows} hidden={hidden} vocab={vocab} chunk={chunk} "
              f"layout={layout} dX={dxt} dW={dwt} beta={beta} seed={seed}", flush=True)
        x = inputs(oracle, (rows, hidden), seed, 1.0, True)
        w = inputs(oracle, (hidden, vocab) if layout == 0 else (vocab, hidden), seed + 1, 0.05, True)
        t = np.random.default_rng(seed).integers(0, vocab, rows).astype(np.int64)
        X, W = to_dev(x, dev, True), to_dev(w, dev, True)
        T = torch.from_numpy(t.astype(np.int32)).to(dev)
        dX = torch.empty((rows, hidden), dtype=tdt[dxt], device=dev) if dxt else None
        dw0 = inputs(oracle, w.shape, seed + 2, 0.01, dwt == "bf16") if dwt else None
        dW = torch.from_numpy(dw0).to(dev, tdt[dwt]) if dwt else None
        loss, row_loss, _ = mi.lm_head_xent(X, W, T, w_layout=layout, chunk=chunk, dX=dX, dW=dW,
                                            dw_beta=beta)
        logits = oracle.round_bf16(oracle.gemm(0, layout, rows, vocab, hidden, x, w).astype(np.float32))
        ref_loss, ref_rows, G = oracle.cross_entropy(logits, t)
        got = host(row_loss)
        err = np.abs(got - ref_rows) / np.maximum(1.0, np.abs(ref_rows))
        assert err.max() <= 2e-3, f"row loss err {err.max():.3e}"
        assert abs(float(loss.item()) - ref_loss) <= 2e-3 * max(1.0, abs(ref_loss))
        g = oracle.round_bf16(G.astype(np.float32))
        if dxt:
            check(host(dX), oracle.gemm(0, 1 - layout, rows, hidden, vocab, g, w), TOL_BF16, "dX")
        if dwt:
            if layout == 0:
                ref = oracle.gemm(1, 0, hidden, vocab, rows, x, g, beta=beta, C0=dw0)
            else:
                ref = oracle.gemm(1, 0, vocab, hidden, rows, g, x, beta=beta, C0=dw0)
            check(host(dW), ref, TOL_BF16, "dW")
