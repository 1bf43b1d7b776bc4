"""The cross-entropy restatement in the oracle (mo_cross_entropy, Loss.cpp:43-195)
pinned without an import of the reference: its known answers (test_loss.cpp
TC-01 .. TC-04, reference_kats.json), scipy's logsumexp / softmax, the two-class
closed form (softplus), and invariants (gradient rows sum to zero, shift
invariance, the 1e-15 clamp)."""
import json
import os

import numpy as np
import pytest
from scipy.special import log_softmax, logsumexp, softmax

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _kats():
    return json.load(open(os.path.join(HERE, "reference_kats.json")))


def test_reference_loss_kats(oracle):
    k = _kats()
    for name in ("loss_tc01", "loss_tc03"):
        c = k[name]
        rows, V = int(np.prod(c["shape"][:-1])), c["shape"][-1]
        loss, row_loss, _ = oracle.cross_entropy(np.full((rows, V), c["logit"]), [c["target"]] * rows)
        assert np.isfinite(loss) and abs(loss - c["expected_loss"]) < c["tol"], name
    c = k["loss_tc02"]
    _, _, grad = oracle.cross_entropy(np.full((1, 4), c["logit"]), [c["target"]])
    assert np.max(np.abs(grad[0] - np.array(c["expected_grad"]))) < c["tol"]
    c = k["loss_tc04"]
    rows, V = int(np.prod(c["shape"][:-1])), c["shape"][-1]
    _, _, grad = oracle.cross_entropy(np.full((rows, V), c["logit"]), [c["target"]] * rows)
    assert list(grad.reshape(c["shape"]).shape) == c["expected_grad_shape"]
    # uniform logits with target 0: every non-target entry is 1/V/rows, the target 1/V/rows - 1/rows
    assert np.allclose(grad[:, 1:], 1.0 / V / rows) and np.allclose(grad[:, 0], (1.0 / V - 1) / rows)


def test_against_scipy(oracle):
    rng = np.random.default_rng(5)
    x = rng.normal(0, 3, (37, 501)).astype(np.float32)
    t = rng.integers(0, 501, 37)
    scale = 0.37
    loss, row_loss, grad = oracle.cross_entropy(x, t, scale=scale)
    xd = x.astype(np.float64)
    ref_rows = logsumexp(xd, axis=1) - xd[np.arange(37), t]
    assert np.allclose(row_loss, ref_rows, rtol=1e-12, atol=1e-12)
    assert np.allclose(row_loss, -log_softmax(xd, axis=1)[np.arange(37), t], rtol=1e-12)
    onehot = np.zeros_like(xd)
    onehot[np.arange(37), t] = 1.0
    assert np.allclose(grad, (softmax(xd, axis=1) - onehot) * scale, rtol=1e-12, atol=1e-15)
    assert abs(loss - ref_rows.sum() * scale) < 1e-9


def test_two_class_closed_form_and_invariants(oracle):
    a = np.array([[2.0, -1.0], [0.5, 3.0], [-4.0, -4.0]], np.float32)
    t = np.array([0, 0, 1])
    _, row_loss, grad = oracle.cross_entropy(a, t, scale=1.0)
    other = a[np.arange(3), 1 - t].astype(np.float64)
    mine = a[np.arange(3), t].astype(np.float64)
    assert np.allclose(row_loss, np.log1p(np.exp(other - mine)), rtol=1e-12)
    assert np.allclose(grad.sum(axis=1), 0.0, atol=1e-15)   # softmax sums to 1, minus the one-hot
    # a constant added to a row changes nothing (the max subtraction, Loss.cpp:95-107)
    _, row_loss2, grad2 = oracle.cross_entropy(a + np.float32(64.0), t, scale=1.0)
    assert np.allclose(row_loss2, row_loss, rtol=1e-12) and np.allclose(grad2, grad, atol=1e-15)


def test_clamp_nan_and_bad_target(oracle):
    # p_target below 1e-15 is clamped (Loss.cpp:115): loss = -log(1e-15f)
    _, row_loss, grad = oracle.cross_entropy(np.array([[0.0, -100.0]]), [1], scale=1.0)
    assert abs(row_loss[0] - (-np.log(np.float64(np.float32(1e-15))))) < 1e-12
    assert np.allclose(grad, [[1.0, -1.0]])
    # just above the clamp: the exact value
    _, row_loss, _ = oracle.cross_entropy(np.array([[0.0, -30.0]]), [1], scale=1.0)
    assert abs(row_loss[0] - np.log1p(np.exp(30.0))) < 1e-12
    _, row_loss, _ = oracle.cross_entropy(np.array([[0.0, np.nan, 1.0]]), [0], scale=1.0)
    assert np.isnan(row_loss[0])
    loss, row_loss, grad = oracle.cross_entropy(np.zeros((2, 3)), [1, 7], scale=0.5)
    assert np.isnan(row_loss[1]) and not np.isnan(row_loss[0])
    assert np.allclose(grad[1], 0.5 / 3)                       # no one-hot term
