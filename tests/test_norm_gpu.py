"""RMSNorm forward / backward (mi_rmsnorm_fwd, mi_rmsnorm_bwd) on the GPU vs the oracle's
restatement of RMSNorm.cpp:40-180 and the decoder layer's fused forms (residual add before
the norm, Transformer.cpp:150-158; residual gradient added to dx, :441-466): every kernel
path (register rows of 1 .. 8 vectors per lane, the generic kernels for long, unaligned or
padded rows), bf16 and fp32 activations and weights, in place, accumulation into dw,
bit-identical dw across launches, and the configuration-3 size (8192 x 2048).

Tolerances (max |got - ref| / max |ref|, ref in float64 from the same input values):
1e-4 for fp32 outputs, 1e-2 for bf16 outputs. The residual sum x + r is stored in x's dtype
and must match the oracle's stored sum bit for bit.
"""
import numpy as np
import pytest

from gpu_cases import TOL_BF16, TOL_F32, check, host

pytestmark = pytest.mark.gpu

# (rows, dims, activation dtype, weight dtype, ld)
CASES = [
    (64, 2048, "bf16", "bf16", None),
    (33, 768, "f32", "f32", None),
    (7, 4096, "bf16", "f32", None),
    (5, 8192, "bf16", "bf16", None),     # longer than the register rows: generic
    (9, 100, "bf16", "bf16", None),      # not whole 16-byte vectors: generic
    (6, 96, "f32", "bf16", 128),         # padded rows, aligned: register kernel
    (6, 96, "bf16", "bf16", 100),        # padded rows, unaligned: generic
    (1, 64, "f32", "f32", None),
    (5000, 256, "bf16", "bf16", None),   # more rows than the backward grid's waves
]


def _tensors(torch, dev, rows, dims, dt, ld, seed, n=3):
    rng = np.random.default_rng(seed)
    out = []
    for k in range(n):
        a = rng.normal(0.0, 1.0 if k != 1 else 0.5, (rows, dims)).astype(np.float32)
        buf = torch.full((rows, ld or dims), 3.0, dtype=dt, device=dev)
        buf[:, :dims] = torch.from_numpy(a).to(dev, dt)
        out.append(buf[:, :dims])
    return out


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("rows,dims,dt_x,dt_w,ld", CASES)
def test_forward_backward_vs_oracle(mi, dev, oracle, rows, dims, dt_x, dt_w, ld):
    import torch

    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}
    tol = TOL_F32 if dt_x == "f32" else TOL_BF16
    print(f"rmsnorm rows={rows} dims={dims} {dt_x}/{dt_w} ld={ld}", flush=True)
    x, r, g = _tensors(torch, dev, rows, dims, tdt[dt_x], ld, 100 + dims + rows)
    w = torch.from_numpy(np.random.default_rng(dims).normal(1.0, 0.2, dims).astype(np.float32))
    w = w.to(dev, tdt[dt_w])
    eps = 1e-5
    xv, rv, gv, wv = _np(x), _np(r), _np(g), _np(w)
    # forward, plain
    rstd = torch.empty((rows,), dtype=torch.float32, device=dev)
    y = mi.rms_norm_forward(x, w, eps, rstd=rstd)
    y_ref, rstd_ref, _ = oracle.rmsnorm_fwd(xv, wv, eps)
    check(host(y), y_ref, tol, "y")
    assert np.allclose(host(rstd), rstd_ref, rtol=1e-5)
    # forward with the residual add: x is updated in place to x + r in its dtype
    x2 = x.clone() if ld is None else _tensors(torch, dev, rows, dims, tdt[dt_x], ld, 100 + dims + rows)[0]
    y2 = mi.rms_norm_forward(x2, w, eps, residual=r)
    y2_ref, _, x_after = oracle.rmsnorm_fwd(xv, wv, eps, residual=rv, round_bf16=dt_x == "bf16")
    assert np.array_equal(_np(x2), x_after), "x + r as stored"
    check(host(y2), y2_ref, tol, "y (residual)")
    # backward with the residual gradient and dw accumulated onto 0.5
    dw = torch.full((dims,), 0.5, dtype=torch.float32, device=dev)
    dx, dw = mi.rms_norm_backward(g, x, w, eps, residual_grad=r, dw=dw, dw_beta=1.0)
    dx_ref, dw_ref = oracle.rmsnorm_bwd(gv, xv, wv, eps, residual_grad=rv, dw0=np.full(dims, 0.5))
    check(host(dx), dx_ref, tol, "dx")
    check(host(dw), dw_ref, TOL_F32 if dt_x == "f32" else 2e-3, "dw")


@pytest.mark.parametrize("dt_x", ["f32", "bf16"])
@pytest.mark.parametrize("dims", [1024, 1000])
def test_in_place_and_determinism(mi, dev, dt_x, dims):
    import torch

    dt = torch.float32 if dt_x == "f32" else torch.bfloat16
    x, r, g = _tensors(torch, dev, 300, dims, dt, None, 7 + dims)
    w = torch.linspace(0.5, 1.5, dims, device=dev).to(dt)
    y = mi.rms_norm_forward(x, w)
    x2 = x.clone()
    y2 = mi.rms_norm_forward(x2, w, out=x2)            # in place
    assert torch.equal(y2, y) and y2.data_ptr() == x2.data_ptr()
    dx1, dw1 = mi.rms_norm_backward(g, x, w, residual_grad=r)
    dx2, dw2 = mi.rms_norm_backward(g, x, w, residual_grad=r)
    assert torch.equal(dx1, dx2) and torch.equal(dw1, dw2)   # fixed-order dw
    g2 = g.clone()
    dx3, dw3 = mi.rms_norm_backward(g2, x, w, residual_grad=r, dx=g2)   # dx over dy
    assert torch.equal(dx3, dx1) and torch.equal(dw3, dw1)
    dx4, none = mi.rms_norm_backward(g, x, w, want_dw=False)
    assert none is None
    dx5, _ = mi.rms_norm_backward(g, x, w)
    assert torch.equal(dx4, dx5)


def test_bf16_weight_gradient_and_mirror(mi, dev, oracle):
    import torch

    x, _, g = _tensors(torch, dev, 64, 512, torch.bfloat16, None, 5)
    norm = mi.RMSNorm(512, eps=1e-5, device=dev)
    norm.weight.copy_(torch.linspace(0.8, 1.2, 512, device=dev).to(torch.bfloat16))
    y = norm.forward(x)
    gw = torch.ones((512,), dtype=torch.float32, device=dev)
    dx = norm.backward(g, x, gw)                       # accumulates into gw
    xv, gv, wv = _np(x), _np(g), _np(norm.weight)
    y_ref, _, _ = oracle.rmsnorm_fwd(xv, wv, 1e-5)
    dx_ref, dw_ref = oracle.rmsnorm_bwd(gv, xv, wv, 1e-5, dw0=np.ones(512))
    check(host(y), y_ref, TOL_BF16, "y")
    check(host(dx), dx_ref, TOL_BF16, "dx")
    check(host(gw), dw_ref, 2e-3, "dw")
    dwb = torch.zeros((512,), dtype=torch.bfloat16, device=dev)   # bf16 weight gradient
    mi.rms_norm_backward(g, x, norm.weight, dw=dwb)
    check(host(dwb), dw_ref - 1.0, TOL_BF16, "dw bf16")
    with pytest.raises(ValueError):
        norm.forward(torch.zeros((4, 256), dtype=torch.bfloat16, device=dev))


def test_config3_size(mi, dev, oracle):
    """The decoder layer's norms at configuration 3: 8192 tokens x 2048, bf16: h += attn_out;
    ffn_in = rmsnorm(h); backward with the residual gradient and dw. Sampled rows against the
    oracle, dw over all rows."""
    import torch

    rows, dims = 8192, 2048
    gen = torch.Generator(device=dev)
    gen.manual_seed(33)
    h = torch.randn((rows, dims), generator=gen, device=dev).to(torch.bfloat16)
    a = torch.randn((rows, dims), generator=gen, device=dev).to(torch.bfloat16)
    dy = (torch.randn((rows, dims), generator=gen, device=dev) * 1e-2).to(torch.bfloat16)
    rg = (torch.randn((rows, dims), generator=gen, device=dev) * 1e-2).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn((dims,), generator=gen, device=dev)).to(torch.bfloat16)
    hv, av, wv = _np(h), _np(a), _np(w)
    y = mi.rms_norm_forward(h, w, 1e-5, residual=a)
    pick = np.array([0, 1, 4097, 8191])
    y_ref, _, h_after = oracle.rmsnorm_fwd(hv[pick], wv, 1e-5, residual=av[pick], round_bf16=True)
    assert np.array_equal(_np(h[pick]), h_after)
    check(host(y[pick]), y_ref, TOL_BF16, "y")
    dx, dw = mi.rms_norm_backward(dy, h, w, 1e-5, residual_grad=rg)
    dx_ref, dw_ref = oracle.rmsnorm_bwd(_np(dy), _np(h), wv, 1e-5, residual_grad=_np(rg))
    check(host(dx[pick]), dx_ref[pick], TOL_BF16, "dx")
    check(host(dw), dw_ref, 1e-3, "dw")


def test_reference_kats(mi, dev):
    """test_rmsnorm.cpp:48-130 (TC-01 .. TC-10) through the RMSNorm mirror, fp32."""
    import json
    import os

    import torch

    k = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                    "reference_kats.json")))
    c = k["rmsnorm_tc03_06"]
    norm = mi.RMSNorm(2, eps=c["eps"], device=dev, dtype=torch.float32)
    assert tuple(norm.weight.shape) == (2,) and torch.all(norm.weight == 1.0)      # TC-01, TC-02
    x = torch.tensor(c["x"], dtype=torch.float32, device=dev)
    y = norm.forward(x).cpu().numpy()
    assert np.max(np.abs(y - np.array(c["expected"]))) < c["tol"]                  # TC-03 .. 06
    c = k["rmsnorm_tc07_08"]
    norm.weight.copy_(torch.tensor(c["weight"], device=dev))
    y = norm.forward(x).cpu().numpy()
    assert np.max(np.abs(y[0] - np.array(c["expected_row0"]))) < c["tol"]          # TC-07, 08
    with pytest.raises(ValueError):                                                # TC-09
        norm.forward(torch.ones((4,), dtype=torch.float32, device=dev))
    with pytest.raises(ValueError):                                                # TC-10
        norm.forward(torch.ones((2, 3), dtype=torch.float32, device=dev))
