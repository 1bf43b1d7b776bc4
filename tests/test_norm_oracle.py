"""The RMSNorm restatement in the oracle (mo_rmsnorm_fwd / mo_rmsnorm_bwd,
RMSNorm.cpp:40-180 and the fused residual forms of Transformer.cpp:150-158,441-466)
pinned without the reference: torch.nn.functional.rms_norm and its autograd
gradients in float64 (library routines), closed forms (constant rows, scale
invariance), central finite differences, and the residual composition."""
import numpy as np
import pytest


def _torch_ref(x, w, eps, dy):
    import torch

    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    y = torch.nn.functional.rms_norm(xt, (x.shape[1],), wt, eps)
    y.backward(torch.tensor(dy, dtype=torch.float64))
    return y.detach().numpy(), xt.grad.numpy(), wt.grad.numpy()


def test_against_torch_rms_norm(oracle):
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, (13, 96)).astype(np.float32)
    w = rng.normal(1, 0.3, 96).astype(np.float32)
    dy = rng.normal(0, 1, (13, 96)).astype(np.float32)
    eps = 1e-5
    y, rstd, _ = oracle.rmsnorm_fwd(x, w, eps)
    dx, dw = oracle.rmsnorm_bwd(dy, x, w, eps)
    ty, tdx, tdw = _torch_ref(x.astype(np.float64), w.astype(np.float64), eps, dy.astype(np.float64))
    assert np.allclose(y, ty, rtol=1e-12, atol=1e-12)
    assert np.allclose(dx, tdx, rtol=1e-10, atol=1e-12)
    assert np.allclose(dw, tdw, rtol=1e-10, atol=1e-12)
    assert np.allclose(rstd, 1 / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1) + eps), rtol=1e-12)


def test_closed_forms(oracle):
    # a constant row c: y = w * c / sqrt(c^2 + eps)
    x = np.full((2, 8), 3.0, np.float32)
    x[1] = -0.5
    w = np.arange(1, 9, dtype=np.float32)
    eps = 1e-2
    y, _, _ = oracle.rmsnorm_fwd(x, w, eps)
    for i, c in enumerate((3.0, -0.5)):
        assert np.allclose(y[i], w * c / np.sqrt(c * c + eps), rtol=1e-12)
    # scale invariance with eps = 0; the gradient of a scale-invariant map is orthogonal to x
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (4, 32)).astype(np.float32)
    w = np.ones(32, np.float32)
    y1, _, _ = oracle.rmsnorm_fwd(x, w, 0.0)
    y2, _, _ = oracle.rmsnorm_fwd(x * np.float32(8.0), w, 0.0)
    assert np.allclose(y1, y2, rtol=1e-12)
    assert np.allclose((y1 ** 2).mean(axis=1), 1.0, rtol=1e-12)
    dy = rng.normal(0, 1, (4, 32)).astype(np.float32)
    dx, _ = oracle.rmsnorm_bwd(dy, x, w, 0.0)
    assert np.allclose((dx * x).sum(axis=1), 0.0, atol=1e-10)


def test_finite_differences(oracle):
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1, (3, 10))
    w = rng.normal(1, 0.2, 10)
    G = rng.normal(0, 1, (3, 10))
    eps = 1e-3

    def loss(xx, ww):
        y, _, _ = oracle.rmsnorm_fwd(xx.astype(np.float32), ww.astype(np.float32), eps)
        return (y * G).sum()

    x32, w32 = x.astype(np.float32).astype(np.float64), w.astype(np.float32).astype(np.float64)
    dx, dw = oracle.rmsnorm_bwd(G.astype(np.float32), x32.astype(np.float32), w32.astype(np.float32), eps)
    h = 1e-2
    for (i, j) in [(0, 0), (1, 4), (2, 9)]:
        xp, xm = x32.copy(), x32.copy()
        xp[i, j] += h
        xm[i, j] -= h
        fd = (loss(xp, w32) - loss(xm, w32)) / (2 * h)
        assert abs(fd - dx[i, j]) < 2e-3 * max(1.0, abs(fd)), (i, j, fd, dx[i, j])
    for j in (0, 5):
        wp, wm = w32.copy(), w32.copy()
        wp[j] += h
        wm[j] -= h
        fd = (loss(x32, wp) - loss(x32, wm)) / (2 * h)
        assert abs(fd - dw[j]) < 2e-3 * max(1.0, abs(fd))


def test_residual_forms(oracle):
    rng = np.random.default_rng(9)
    x = rng.normal(0, 1, (5, 16)).astype(np.float32)
    r = rng.normal(0, 1, (5, 16)).astype(np.float32)
    w = rng.normal(1, 0.1, 16).astype(np.float32)
    y, _, x_after = oracle.rmsnorm_fwd(x, w, 1e-5, residual=r)
    y_ref, _, _ = oracle.rmsnorm_fwd(x + r, w, 1e-5)
    assert np.array_equal(x_after, x + r) and np.allclose(y, y_ref, rtol=1e-12)
    # bf16 storage: the norm sees the rounded sum
    _, _, xb = oracle.rmsnorm_fwd(x, w, 1e-5, residual=r, round_bf16=True)
    assert np.array_equal(xb, oracle.round_bf16(x + r))
    dy = rng.normal(0, 1, (5, 16)).astype(np.float32)
    g = rng.normal(0, 1, (5, 16)).astype(np.float32)
    dx, dw = oracle.rmsnorm_bwd(dy, x, w, 1e-5, residual_grad=g, dw0=np.ones(16))
    dx0, dw0 = oracle.rmsnorm_bwd(dy, x, w, 1e-5)
    assert np.allclose(dx, dx0 + g, rtol=1e-12) and np.allclose(dw, dw0 + 1.0, rtol=1e-12)


def test_reference_kats(oracle):
    """test_rmsnorm.cpp:48-130: x = [[0.3, 0.9], [-0.7, 0.4]], eps 1e-5, unit and [2, 0.5] weights."""
    import json
    import os

    k = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                    "reference_kats.json")))
    c = k["rmsnorm_tc03_06"]
    y, _, _ = oracle.rmsnorm_fwd(np.array(c["x"], np.float32), np.array(c["weight"], np.float32), c["eps"])
    assert np.max(np.abs(y - np.array(c["expected"]))) < c["tol"]
    c = k["rmsnorm_tc07_08"]
    y, _, _ = oracle.rmsnorm_fwd(np.array(c["x"], np.float32), np.array(c["weight"], np.float32), c["eps"])
    assert np.max(np.abs(y[0] - np.array(c["expected_row0"]))) < c["tol"]
