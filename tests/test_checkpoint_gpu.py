"""Checkpoint weights loaded onto the GPU (mi_gemm.load_weights over mi_convert_matrix) vs
the oracle's restatement of the reference loader (Checkpoint.cpp:28-83, 390-570): a
Python/MLX file with bf16, f16 and fp32 tensors (transposed [out, in] matrices, de-fused
wqkv and w12) and engine files, into fp32 (exact) and bf16 (round to nearest even of the
exact value) buffers; odd-shaped slices and transposes; missing and mismatched tensors."""
import numpy as np
import pytest

from checkpoint_files import CFG, write_engine_file, write_python_file

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fmt", ["python", "engine_f32", "engine_bf16"])
@pytest.mark.parametrize("dst", ["f32", "bf16"])
def test_load_weights(mi, dev, oracle, tmp_path, fmt, dst):
    import torch

    path = str(tmp_path / f"{fmt}.safetensors")
    if fmt == "python":
        write_python_file(path)
    else:
        write_engine_file(path, dtype=torch.float32 if fmt == "engine_f32" else torch.bfloat16)
    print(f"load_weights {fmt} -> {dst}", flush=True)
    w = mi.load_weights(path, CFG, dtype=torch.float32 if dst == "f32" else torch.bfloat16, device=dev)
    ref = oracle.checkpoint_weights(path, CFG)
    assert set(w) == set(ref)
    for k, v in ref.items():
        got = w[k].float().cpu().numpy()
        want = v if dst == "f32" else oracle.round_bf16(v)
        assert got.shape == want.shape and np.array_equal(got, want), k


@pytest.mark.parametrize("src_dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("R,C,row0,rows", [(130, 77, 5, 100),     # element-wise paths
                                          (130, 96, 4, 100),     # 8-element copy, 4-element transpose
                                          (130, 100, 4, 100),    # 4-element copy
                                          (200, 192, 8, 192),    # interior transpose tiles
                                          (70000, 8, 0, 70000)])  # more rows than a grid column
def test_convert_matrix_slices(mi, dev, src_dt, transpose, R, C, row0, rows):
    import torch

    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[src_dt]
    code = {"f32": mi.MI_F32, "bf16": mi.MI_BF16, "f16": mi.MI_F16}[src_dt]
    print(f"convert {src_dt} {R}x{C} rows {row0}+{rows} transpose={transpose}", flush=True)
    src = torch.randn((R, C), device=dev).to(tdt)
    for out_dt in (torch.float32, torch.bfloat16):
        dst = torch.full((C, rows) if transpose else (rows, C), 7.0, dtype=out_dt, device=dev)
        mi.convert_matrix(src, code, C, row0, rows, C, transpose, dst)
        want = src[row0:row0 + rows].float()
        want = (want.t() if transpose else want).to(out_dt)
        assert torch.equal(dst, want)


@pytest.mark.parametrize("transpose", [False, True])
def test_convert_matrix_padded_destination(mi, dev, transpose):
    """A destination leading dimension above its row length (the 4-element copy and
    transpose paths): the rows land at dst_ld apart and the pad columns keep their values."""
    import torch

    R, C = 64, 96
    src = torch.randn((R, C), device=dev).to(torch.bfloat16)
    drows, dcols = (C, R) if transpose else (R, C)
    ld = dcols + 8
    dst = torch.full((drows, ld), 7.0, dtype=torch.bfloat16, device=dev)
    st = mi.load_library().mi_convert_matrix(mi._stream(), mi._ptr(src), mi.MI_BF16, C, 0, R, C,
                                             int(transpose), mi._ptr(dst), mi.MI_BF16, ld)
    torch.cuda.synchronize()
    assert st == 0
    want = src.t() if transpose else src
    assert torch.equal(dst[:, :dcols], want)
    assert torch.all(dst[:, dcols:] == 7.0)


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("R,C,row0,rows", [(200, 192, 8, 192), (130, 77, 5, 100), (130, 100, 4, 100)])
def test_convert_matrix_bf16_bits_exact(mi, dev, transpose, R, C, row0, rows):
    """bf16 -> bf16 moves every bit pattern unchanged, NaN payloads and signalling NaNs
    included, on the interior-tile, edge and copy paths."""
    import torch

    print(f"convert bf16 bits {R}x{C} rows {row0}+{rows} transpose={transpose}", flush=True)
    g = torch.Generator().manual_seed(R * C + rows)
    bits = torch.randint(-32768, 32768, (R, C), generator=g, dtype=torch.int32).to(torch.int16)
    bits[0, :8] = torch.tensor([0x7f81, 0x7fc1, -0x7f, -0x3f, 0x7f80, -0x80, 0x0001, -0x8000],
                               dtype=torch.int16)  # sNaN, qNaN, -sNaN, -qNaN, +-inf, subnormal, -0
    src = bits.to(dev).view(torch.bfloat16)
    dst = torch.zeros((C, rows) if transpose else (rows, C), dtype=torch.bfloat16, device=dev)
    mi.convert_matrix(src, mi.MI_BF16, C, row0, rows, C, transpose, dst)
    want = bits[row0:row0 + rows]
    want = want.t() if transpose else want
    assert torch.equal(dst.view(torch.int16).cpu(), want.contiguous())


def test_missing_and_mismatched(mi, dev, tmp_path):
    import torch
    from safetensors.torch import save_file

    path = str(tmp_path / "mlx.safetensors")
    tensors = write_python_file(path)
    del tensors["layers.1.feed_forward.w12.weight"]
    p2 = str(tmp_path / "missing.safetensors")
    save_file(tensors, p2)
    with pytest.raises(KeyError):
        mi.load_weights(p2, CFG, device=dev)
    tensors["layers.1.feed_forward.w12.weight"] = torch.zeros((10, 64))
    p3 = str(tmp_path / "shape.safetensors")
    save_file(tensors, p3)
    with pytest.raises(ValueError):
        mi.load_weights(p3, CFG, device=dev)
