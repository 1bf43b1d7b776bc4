"""Seeded sweeps of the residual add + RMSNorm kernels (RMSNorm.cpp:40-180, Transformer.cpp:
150-158 and 441-466) and the softmax cross-entropy (Loss.cpp:43-195) over random shapes:
row counts from 1 to a few thousand, row lengths on and off whole 16-byte vectors and on
either side of the register-row limits, bf16 and fp32 activations, weights, logits and
gradients, packed and padded rows (aligned and unaligned leading dimensions).  Every case
is checked against the oracle at the tolerances of test_norm_gpu.py / test_xent_gpu.py.
"""
import numpy as np
import pytest

from gpu_cases import TOL_BF16, TOL_F32, check, host

pytestmark = pytest.mark.gpu


def _pad(rng, n):
    """None (packed rows) or a leading dimension past n: a multiple of 8 or not."""
    k = int(rng.integers(0, 3))
    if k == 0:
        return None
    if k == 1:
        return n + 8 * int(rng.integers(1, 9)) - n % 8
    return n + int(rng.integers(1, 9))


def _norm_cases(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        rows = int(rng.choice([1, 2, 7, 33, 130, 513, 2049, 4100]))
        dims = int(rng.choice([8 * int(rng.integers(1, 1025)), int(rng.integers(1, 1200))]))
        out.append((rows, dims, str(rng.choice(["bf16", "f32"])), str(rng.choice(["bf16", "f32"])),
                    _pad(rng, dims), int(rng.integers(1 << 20))))
    return out


def _rows(torch, dev, rng, rows, dims, dt, ld, std):
    a = rng.normal(0.0, std, (rows, dims)).astype(np.float32)
    buf = torch.full((rows, ld or dims), 3.0, dtype=dt, device=dev)
    buf[:, :dims] = torch.from_numpy(a).to(dev, dt)
    return buf[:, :dims]


@pytest.mark.parametrize("part", range(3))
def test_rmsnorm_sweep(mi, dev, oracle, part):
    import torch

    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}
    for rows, dims, dt_x, dt_w, ld, seed in _norm_cases(8100 + part, 12):
        print(f"rmsnorm sweep rows={rows} dims={dims} {dt_x}/{dt_w} ld={ld} seed={seed}", flush=True)
        rng = np.random.default_rng(seed)
        tol = TOL_F32 if dt_x == "f32" else TOL_BF16
        x = _rows(torch, dev, rng, rows, dims, tdt[dt_x], ld, 1.0)
        r = _rows(torch, dev, rng, rows, dims, tdt[dt_x], ld, 0.5)
        g = _rows(torch, dev, rng, rows, dims, tdt[dt_x], ld, 1.0)
        w = torch.from_numpy(rng.normal(1.0, 0.2, dims).astype(np.float32)).to(dev, tdt[dt_w])
        eps = 1e-5
        xv, rv, gv, wv = (t.float().cpu().numpy() for t in (x, r, g, w))
        y = mi.rms_norm_forward(x, w, eps)
        y_ref, _, _ = oracle.rmsnorm_fwd(xv, wv, eps)
        check(host(y), y_ref, tol, "y")
        x2 = torch.empty_strided(x.shape, x.stride(), dtype=x.dtype, device=dev)   # x's row stride
        x2.copy_(x)
        y2 = mi.rms_norm_forward(x2, w, eps, residual=r)
        y2_ref, _, x_after = oracle.rmsnorm_fwd(xv, wv, eps, residual=rv, round_bf16=dt_x == "bf16")
        assert np.array_equal(x2.float().cpu().numpy(), x_after), "x + r as stored"
        check(host(y2), y2_ref, tol, "y (residual)")
        dw = torch.full((dims,), 0.25, dtype=torch.float32, device=dev)
        dx, dw = mi.rms_norm_backward(g, x, w, eps, residual_grad=r, dw=dw, dw_beta=1.0)
        dx_ref, dw_ref = oracle.rmsnorm_bwd(gv, xv, wv, eps, residual_grad=rv, dw0=np.full(dims, 0.25))
        check(host(dx), dx_ref, tol, "dx")
        check(host(dw), dw_ref, TOL_F32 if dt_x == "f32" else 2e-3, "dw")


def _xent_cases(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        rows = int(rng.choice([1, 3, 8, 17, 64, 129, 300]))
        V = int(rng.choice([8 * int(rng.integers(1, 8001)), int(rng.integers(2, 40000))]))
        out.append((rows, V, str(rng.choice(["bf16", "f32"])), str(rng.choice(["bf16", "f32"])),
                    _pad(rng, V), int(rng.integers(1 << 20))))
    return out


@pytest.mark.parametrize("part", range(3))
def test_cross_entropy_sweep(mi, dev, oracle, part):
    import torch

    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}
    for rows, V, dt_in, dt_out, ld, seed in _xent_cases(8200 + part, 12):
        print(f"cross_entropy sweep rows={rows} V={V} {dt_in}->{dt_out} ld={ld} seed={seed}", flush=True)
        rng = np.random.default_rng(seed)
        x = rng.normal(0.0, 2.0, (rows, V)).astype(np.float32)
        if rows > 1:
            x[0] *= 20.0   # a wide row
        buf = torch.full((rows, ld or V), -7.0, dtype=tdt[dt_in], device=dev)   # padding is ignored
        buf[:, :V] = torch.from_numpy(x).to(dev, tdt[dt_in])
        L = buf[:, :V]
        xv = L.float().cpu().numpy()
        t = rng.integers(0, V, rows)
        T = torch.from_numpy(t).to(dev)
        loss, row_loss, grad = mi.cross_entropy(L, T, grad_dtype=tdt[dt_out])
        ref_loss, ref_rows, ref_grad = oracle.cross_entropy(xv, t)
        got = host(row_loss)
        err = np.abs(got - ref_rows) / np.maximum(1.0, np.abs(ref_rows))
        assert err.max() <= 1e-5, f"row loss err {err.max():.3e}"
        assert abs(loss.item() - ref_loss) <= 1e-5 * max(1.0, abs(ref_loss))
        check(host(grad), ref_grad, TOL_F32 if dt_out == "f32" else TOL_BF16, "grad")
