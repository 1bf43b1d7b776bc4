"""Softmax cross-entropy (mi_cross_entropy) on the GPU vs the oracle's restatement of
CrossEntropyLoss (Loss.cpp:43-195): the reference's known answers (test_loss.cpp
TC-01 .. TC-04), seeded rows of every kernel path (register-resident rows of 1 .. 16
vectors per thread, the streaming kernel for long or unaligned rows, padded leading
dimensions, bf16 and fp32 logits and gradients, in place), out-of-range targets, the
1e-15 clamp, determinism, and the configuration-5 size (8192 x 32000).

Tolerances: both sides see the same logit values (bf16-rounded where the logits are
bf16). Row losses: |got - ref| <= 1e-5 * max(1, |ref|) (the 1e-5 of TC-01 / TC-03).
Gradients: max |got - ref| / max |ref| <= 1e-4 for fp32 gradients, 1e-2 for bf16.
"""
import json
import os

import numpy as np
import pytest

from gpu_cases import TOL_BF16, TOL_F32, check, host

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _loss_close(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "NaN rows differ"
    ok = ~np.isnan(ref)
    err = np.abs(got[ok] - ref[ok]) / np.maximum(1.0, np.abs(ref[ok]))
    assert err.size == 0 or err.max() <= 1e-5, f"row loss err {err.max():.3e}"


def _logits(rows, V, seed, std=2.0):
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, std, (rows, V)).astype(np.float32)
    if rows > 2:
        x[1] *= 25.0             # wide row: the max subtraction matters
        x[2] += 1000.0           # large offset (TC-03's regime)
    return x


def _dev(torch, x, dt, dev, ld=None):
    rows, V = x.shape
    ld = ld or V
    buf = torch.full((rows, ld), -7.0, dtype=dt, device=dev)   # padding must be ignored
    buf[:, :V] = torch.from_numpy(x).to(dev, dt)
    return buf[:, :V]


@pytest.mark.parametrize("dt_in", ["f32", "bf16"])
def test_reference_kats(mi, dev, dt_in):
    import torch

    k = json.load(open(os.path.join(HERE, "reference_kats.json")))
    dt = torch.float32 if dt_in == "f32" else torch.bfloat16
    loss_fn = mi.CrossEntropyLoss()
    for name in ("loss_tc01", "loss_tc03"):
        c = k[name]
        logits = torch.full(c["shape"], c["logit"], dtype=dt, device=dev)
        targets = torch.full(c["shape"][:-1], c["target"], dtype=torch.int64, device=dev)
        loss = loss_fn.forward(logits, targets)
        assert np.isfinite(loss) and abs(loss - c["expected_loss"]) < c["tol"], (name, loss)
    c = k["loss_tc02"]
    logits = torch.full(c["shape"], c["logit"], dtype=dt, device=dev)
    targets = torch.full(c["shape"][:-1], c["target"], dtype=torch.int64, device=dev)
    loss_fn.forward(logits, targets)
    grad = loss_fn.backward(targets).cpu().numpy()
    assert np.max(np.abs(grad.reshape(-1) - np.array(c["expected_grad"]))) < c["tol"]
    c = k["loss_tc04"]
    logits = torch.full(c["shape"], c["logit"], dtype=dt, device=dev)
    targets = torch.full(c["shape"][:-1], c["target"], dtype=torch.int64, device=dev)
    loss_fn.forward(logits, targets)
    assert list(loss_fn.backward(targets).shape) == c["expected_grad_shape"]


# (rows, V, logits dtype, grad dtype, ld): register rows of 1, 2, 8, 16 vectors per
# thread; 65536 bf16 = exactly 16; streaming for V % 8 != 0, V > 65536 and an
# unaligned leading dimension; padded aligned rows stay on the vector kernel.
CASES = [
    (64, 1000, "bf16", "f32", None),
    (33, 4096, "f32", "f32", None),
    (16, 32000, "bf16", "bf16", None),
    (8, 32000, "f32", "bf16", None),
    (3, 65536, "bf16", "f32", None),
    (7, 33, "bf16", "f32", None),
    (5, 70000, "bf16", "bf16", None),
    (9, 1000, "bf16", "f32", 1024),
    (9, 1000, "bf16", "f32", 1003),
    (6, 999, "f32", "f32", 1001),
]


@pytest.mark.parametrize("rows,V,dt_in,dt_out,ld", CASES)
def test_rows_vs_oracle(mi, dev, oracle, rows, V, dt_in, dt_out, ld):
    import torch

    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}
    x = _logits(rows, V, 7000 + V + rows)
    L = _dev(torch, x, tdt[dt_in], dev, ld)
    xv = L.float().cpu().numpy()                     # the values the kernel sees
    rng = np.random.default_rng(V)
    t = rng.integers(0, V, rows)
    t[0] = V - 1
    T = torch.from_numpy(t).to(dev)
    print(f"cross_entropy rows={rows} V={V} {dt_in}->{dt_out} ld={ld}", flush=True)
    loss, row_loss, grad = mi.cross_entropy(L, T, grad_dtype=tdt[dt_out])
    ref_loss, ref_rows, ref_grad = oracle.cross_entropy(xv, t)
    _loss_close(host(row_loss), ref_rows)
    assert abs(loss.item() - ref_loss) <= 1e-5 * max(1.0, abs(ref_loss))
    check(host(grad), ref_grad, TOL_F32 if dt_out == "f32" else TOL_BF16, "grad")


@pytest.mark.parametrize("dt_in", ["f32", "bf16"])
@pytest.mark.parametrize("V", [4000, 4001])
def test_in_place_and_determinism(mi, dev, dt_in, V):
    import torch

    dt = torch.float32 if dt_in == "f32" else torch.bfloat16
    x = _logits(12, V, 77 + V)
    L = torch.from_numpy(x).to(dev, dt)
    T = torch.from_numpy(np.arange(12) * 331 % V).to(dev)
    loss1, rows1, g1 = mi.cross_entropy(L, T, grad_dtype=dt)
    loss2, rows2, g2 = mi.cross_entropy(L, T, grad_dtype=dt)
    assert torch.equal(loss1, loss2) and torch.equal(rows1, rows2) and torch.equal(g1, g2)
    L2 = L.clone()
    loss3, rows3, g3 = mi.cross_entropy(L2, T, grad="inplace")
    assert g3.data_ptr() == L2.data_ptr()
    assert torch.equal(loss3, loss1) and torch.equal(rows3, rows1) and torch.equal(L2, g1)


def test_clamp_bad_target_and_loss_only(mi, dev, oracle):
    import torch

    x = np.zeros((4, 64), np.float32)
    x[0, 5] = -100.0          # p_target ~ 1e-44 < 1e-15: clamped
    x[1, :] = 3.0
    x[3, 9] = np.nan
    t = np.array([5, 64, 2, 0])   # row 1: target out of range
    L = torch.from_numpy(x).to(dev)
    loss, row_loss, grad = mi.cross_entropy(L, torch.from_numpy(t).to(dev), scale=0.5)
    _, ref_rows, ref_grad = oracle.cross_entropy(x, t, scale=0.5)
    got = host(row_loss)
    _loss_close(got, ref_rows)
    assert abs(got[0] - (-np.log(np.float64(np.float32(1e-15))))) < 1e-5
    g = host(grad)
    assert np.allclose(g[1], 0.5 / 64)              # no one-hot term for the bad target
    assert np.isnan(g[3]).all()                     # NaN logits propagate
    check(g[[0, 2]], ref_grad[[0, 2]], TOL_F32, "grad")
    loss2, rows2, none = mi.cross_entropy(L, torch.from_numpy(t).to(dev), grad=None, scale=0.5)
    assert none is None and np.array_equal(np.isnan(host(rows2)), np.isnan(got))


def test_config5_size(mi, dev, oracle):
    """Configuration 5's loss: 8192 rows of 32000 bf16 logits. Sampled rows against the
    oracle; at full size every gradient row sums to 0 and the loss is the mean row loss."""
    import torch

    rows, V = 8192, 32000
    g = torch.Generator(device=dev)
    g.manual_seed(55)
    L = torch.randn((rows, V), generator=g, device=dev).to(torch.bfloat16)
    T = torch.randint(0, V, (rows,), generator=g, device=dev)
    pick = np.array([0, 1, 777, 4095, 8191])
    xs = L[pick].float().cpu().numpy()
    loss, row_loss, grad = mi.cross_entropy(L, T)                 # fp32 gradient
    ref_loss, ref_rows, ref_grad = oracle.cross_entropy(xs, T[pick].cpu().numpy(), scale=1.0 / rows)
    _loss_close(host(row_loss)[pick], ref_rows)
    check(host(grad[pick]), ref_grad, TOL_F32, "grad")
    sums = grad.double().sum(dim=1).abs().max().item()
    assert sums < 1e-9, sums                                       # sum_v (p - onehot) = 0
    mean = host(row_loss).mean()
    assert abs(loss.item() - mean) <= 1e-5 * mean
    # in place in bf16, as the LM-head step runs it: equal to the out-of-place bf16 gradient
    loss_b, rows_b, gb = mi.cross_entropy(L, T, grad_dtype=torch.bfloat16)
    L2 = L.clone()
    mi.cross_entropy(L2, T, grad="inplace")
    assert torch.equal(L2, gb)
    check(host(gb[pick]), ref_grad, TOL_BF16, "bf16 grad")
