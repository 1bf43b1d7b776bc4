"""LM head + softmax cross-entropy over vocabulary chunks (mi_lm_head_xent): the
reference's logits = final_h.matmul(output_projection_) (Transformer.cpp:193-194), its
CrossEntropyLoss (Loss.cpp:43-195) and the output projection's backward
(Transformer.cpp:600-616), computed without the [rows, vocab] logits.

Checks, for both weight layouts (0: W [hidden, vocab], the reference's; 1: W [vocab, hidden],
a tied table), several chunk sizes (whole 16-byte chunks, chunks that are not, a single
chunk) and dX / dW dtypes:
  * against the oracle: logits = X W rounded to bf16 as the GEMM stores them, then the
    oracle's cross-entropy (row losses, mean loss, gradient G rounded to bf16), dX = G W^T
    and dW = beta dW0 + X^T G in float64;
  * against the unfused library path on the GPU (mi_gemm logits, mi_cross_entropy in place,
    the dX and dW GEMMs), at small sizes and at configuration 5 (8192 x 2048 -> 32000);
  * that results do not depend on the chunk size beyond summation order, and that two calls
    give identical bits.
Tolerances: row losses 2e-3 * max(1, |ref|) against the oracle (the GPU's fp32-accumulated
logit can round to the neighbouring bf16 value, moving the loss by up to one bf16 ulp of a
logit, 0.4 % of its size), the same against the unfused GPU path at configuration 5 (the
full-width logits GEMM and the chunk GEMMs run different tile plans, whose per-XCD K rotation
sums K in another order, so a logit can round to the other neighbouring bf16 value), 1e-5
where both plans are the same (small sizes: only the order of the sum of exponentials
differs); dX and dW max |got - ref| / max |ref| <= 1e-2 (bf16 inputs and gradient).
"""
import numpy as np
import pytest

from gpu_cases import TOL_BF16, check, host, inputs, sample_rows, to_dev

pytestmark = pytest.mark.gpu


def _loss_close(got, ref, tol):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "NaN rows differ"
    ok = ~np.isnan(ref)
    err = np.abs(got[ok] - ref[ok]) / np.maximum(1.0, np.abs(ref[ok]))
    assert err.size == 0 or err.max() <= tol, f"row loss err {err.max():.3e} > {tol:.0e}"


def _problem(oracle, rows, hidden, vocab, layout, seed):
    x = inputs(oracle, (rows, hidden), seed, 1.0, True)
    wshape = (hidden, vocab) if layout == 0 else (vocab, hidden)
    w = inputs(oracle, wshape, seed + 1, 0.05, True)
    t = np.random.default_rng(seed).integers(0, vocab, rows).astype(np.int64)
    return x, w, t


def _tensors(dev, x, w, t):
    import torch

    return to_dev(x, dev, True), to_dev(w, dev, True), torch.from_numpy(t.astype(np.int32)).to(dev)


# rows, hidden, vocab, chunk, layout, dX dtype, dW dtype, dw_beta
CASES = [
    (96, 128, 1000, 256, 0, "bf16", "f32", 1.0),   # 4 chunks (tail 232), reference layout, dW += ...
    (96, 128, 1000, 256, 1, "f32", "f32", 0.0),    # tied layout, fp32 dX (accumulated in place)
    (64, 256, 777, 100, 0, "bf16", "bf16", 0.0),   # chunks and vocab not whole 16-byte vectors
    (130, 64, 4096, 0, 1, "bf16", None, 0.0),      # one chunk: no recomputation; no dW
    (50, 96, 3000, 1024, 1, None, "f32", 1.0),     # dW only
    (33, 128, 2000, 512, 0, None, None, 0.0),      # loss only (pass 1 alone)
    (256, 256, 4096, 1024, 0, "bf16", "f32", 1.0),  # whole 64-column slices everywhere
    (320, 128, 3040, 960, 1, "f32", "bf16", 0.0),   # tail chunk of 160 columns
    (256, 128, 2048, 0, 1, None, None, 0.0),        # one chunk, loss only
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_lm_head_xent_vs_oracle(mi, dev, oracle, case):
    import torch

    rows, hidden, vocab, chunk, layout, dxt, dwt, beta = CASES[case]
    print(f"lm_head_xent rows={rows} hidden={hidden} vocab={vocab} chunk={chunk} layout={layout} "
          f"dX={dxt} dW={dwt} beta={beta}", flush=True)
    x, w, t = _problem(oracle, rows, hidden, vocab, layout, 900 + case)
    if case == 0:
        t[5] = vocab + 3  # a target outside [0, vocab): NaN row loss, no one-hot term
    X, W, T = _tensors(dev, x, w, t)
    tdt = {"bf16": torch.bfloat16, "f32": torch.float32}
    dX = torch.empty((rows, hidden), dtype=tdt[dxt], device=dev) if dxt else None
    dw0 = inputs(oracle, w.shape, 950 + case, 0.01, dwt == "bf16") if dwt else None
    dW = torch.from_numpy(dw0).to(dev, tdt[dwt]) if dwt else None
    loss, row_loss, _ = mi.lm_head_xent(X, W, T, w_layout=layout, chunk=chunk, dX=dX, dW=dW,
                                        dw_beta=beta)
    # oracle: bf16 logits, cross-entropy, bf16 gradient, then the two products
    logits = oracle.round_bf16(oracle.gemm(0, layout, rows, vocab, hidden, x, w).astype(np.float32))
    ref_loss, ref_rows, G = oracle.cross_entropy(logits, t)
    _loss_close(host(row_loss), ref_rows, 2e-3)
    if np.isfinite(ref_loss):
        assert abs(float(loss.item()) - ref_loss) <= 2e-3 * max(1.0, abs(ref_loss))
    else:
        assert np.isnan(loss.item())
    g = oracle.round_bf16(G.astype(np.float32))
    if dxt:
        ref = oracle.gemm(0, 1 - layout, rows, hidden, vocab, g, w)  # G W^T (0) or G W (1)
        check(host(dX), ref, TOL_BF16, "dX vs oracle")
    if dwt:
        if layout == 0:   # dW [hidden, vocab] = beta dW0 + X^T G
            ref = oracle.gemm(1, 0, hidden, vocab, rows, x, g, beta=beta, C0=dw0)
        else:             # dW [vocab, hidden] = beta dW0 + G^T X
            ref = oracle.gemm(1, 0, vocab, hidden, rows, g, x, beta=beta, C0=dw0)
        check(host(dW), ref, TOL_BF16, "dW vs oracle")


def _unfused(mi, X, W, T, layout, dw_beta=0.0, dW=None):
    """The library's separate path: logits GEMM (bf16), cross-entropy in place, dX, dW."""
    import torch

    rows, hidden = X.shape
    vocab = W.shape[1] if layout == 0 else W.shape[0]
    L = torch.empty((rows, vocab), dtype=torch.bfloat16, device=X.device)
    mi.gemm(X, W, L, rows, vocab, hidden, transB=bool(layout))
    loss, row_loss, _ = mi.cross_entropy(L, T, grad="inplace")
    dX = torch.empty((rows, hidden), dtype=torch.bfloat16, device=X.device)
    mi.gemm(L, W, dX, rows, hidden, vocab, transB=not layout)
    if dW is not None:
        if layout == 0:
            mi.gemm(X, L, dW, hidden, vocab, rows, transA=True, beta=dw_beta)
        else:
            mi.gemm(L, X, dW, vocab, hidden, rows, transA=True, beta=dw_beta)
    return loss, row_loss, dX


@pytest.mark.parametrize("layout", [0, 1])
def test_lm_head_xent_vs_unfused_small(mi, dev, oracle, layout):
    import torch

    rows, hidden, vocab = 256, 512, 5000
    x, w, t = _problem(oracle, rows, hidden, vocab, layout, 970 + layout)
    X, W, T = _tensors(dev, x, w, t)
    dW1 = torch.zeros(W.shape, dtype=torch.float32, device=dev)
    dW2 = torch.zeros_like(dW1)
    l1, r1, dX1 = mi.lm_head_xent(X, W, T, w_layout=layout, chunk=1536, dW=dW1, dw_beta=1.0)
    l2, r2, dX2 = _unfused(mi, X, W, T, layout, 1.0, dW2)
    _loss_close(host(r1), host(r2), 1e-5)
    check(host(dX1), host(dX2), TOL_BF16, "dX vs unfused")
    check(host(dW1), host(dW2), TOL_BF16, "dW vs unfused")


def test_chunk_size_and_determinism(mi, dev, oracle):
    """Chunks of 8192, 2048 and one chunk agree; repeated calls give the same bits."""
    rows, hidden, vocab = 512, 256, 20000
    x, w, t = _problem(oracle, rows, hidden, vocab, 1, 990)
    X, W, T = _tensors(dev, x, w, t)
    outs = {}
    for chunk in (8192, 2048, 0):
        outs[chunk] = [host(v) for v in mi.lm_head_xent(X, W, T, w_layout=1, chunk=chunk)]
    for chunk in (2048, 0):
        _loss_close(outs[chunk][1], outs[8192][1], 1e-5)
        check(outs[chunk][2], outs[8192][2], TOL_BF16, f"dX chunk {chunk} vs 8192")
    again = [host(v) for v in mi.lm_head_xent(X, W, T, w_layout=1, chunk=2048)]
    for a, b in zip(again, outs[2048]):
        assert np.array_equal(a, b), "not deterministic"


@pytest.mark.parametrize("layout", [1, 0])
def test_lm_head_xent_config5(mi, dev, oracle, layout):
    """Configuration 5 (8192 x 2048 -> 32000, chunks of 8192): against the unfused path in
    full, and sampled rows of the row losses and dX against the oracle."""
    import torch

    rows, hidden, vocab = 8192, 2048, 32000
    x, w, t = _problem(oracle, rows, hidden, vocab, layout, 995 + layout)
    X, W, T = _tensors(dev, x, w, t)
    dW1 = torch.zeros(W.shape, dtype=torch.float32, device=dev)
    l1, r1, dX1 = mi.lm_head_xent(X, W, T, w_layout=layout, chunk=8192, dW=dW1)
    r1h, dX1h, dW1h = host(r1), host(dX1), host(dW1)
    del dW1
    dW2 = torch.zeros(W.shape, dtype=torch.float32, device=dev)
    l2, r2, dX2 = _unfused(mi, X, W, T, layout, 0.0, dW2)
    _loss_close(r1h, host(r2), 2e-3)
    assert abs(l1.item() - l2.item()) <= 1e-4 * abs(l2.item())
    check(dX1h, host(dX2), TOL_BF16, "dX vs unfused")
    check(dW1h, host(dW2), TOL_BF16, "dW vs unfused")
    sr = sample_rows(rows, 6, 5)
    logits = oracle.round_bf16(oracle.gemm(0, layout, len(sr), vocab, hidden, x[sr], w).astype(np.float32))
    _, ref_rows, G = oracle.cross_entropy(logits, t[sr], scale=1.0 / rows)
    _loss_close(r1h[sr], ref_rows, 2e-3)
    g = oracle.round_bf16(G.astype(np.float32))
    ref = oracle.gemm(0, 1 - layout, len(sr), hidden, vocab, g, w)
    check(dX1h[sr], ref, TOL_BF16, "sampled dX rows vs oracle")
