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
                                          (130, 96, 4, 100),     # 8-element copy, edge tiles
                                          (130, 100, 4, 100),    # 4-element copy
                                          (300, 520, 8, 260),    # interior 64 x 256 tiles, 8-element runs
                                          (130, 516, 4, 100),    # interior tiles, 4-element runs
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
@pytest.mark.parametrize("R,C,row0,rows", [(300, 520, 8, 260), (130, 516, 4, 100), (130, 77, 5, 100),
                                          (130, 100, 4, 100)])
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


def test_convert_matrices_mixed(mi, dev):
    """One mi_convert_matrices call over jobs of every dtype pair, transposed and not,
    interior and edge tiles, shared fused sources, a padded destination and more jobs
    than one launch holds, against the same conversions done one by one."""
    import torch

    torch.manual_seed(5)
    codes = {torch.float32: mi.MI_F32, torch.bfloat16: mi.MI_BF16, torch.float16: mi.MI_F16}
    fused = torch.randn((200, 512), device=dev).to(torch.bfloat16)     # a wqkv-like source
    srcs = [torch.randn((R, C), device=dev).to(dt) for R, C, dt in
            [(130, 77, torch.float32), (96, 100, torch.float16), (64, 64, torch.bfloat16),
             (257, 40, torch.float32), (70, 130, torch.float16), (140, 520, torch.float32),
             (133, 516, torch.bfloat16)]]
    jobs, want = [], []

    def add(src, row0, rows, tr, out_dt, pad=0):
        C = src.shape[1]
        shape = (C, rows + pad) if tr else (rows, C + pad)
        dst = torch.full(shape, 7.0, dtype=out_dt, device=dev)
        view = dst[:, :rows] if tr else dst[:, :C]
        jobs.append((src, codes[src.dtype], C, row0, rows, C, tr, view))
        w = src[row0:row0 + rows].float()
        want.append((dst, (w.t() if tr else w).to(out_dt), pad))

    for row0, rows in ((0, 128), (128, 36), (164, 36)):                 # de-fused row ranges
        add(fused, row0, rows, True, torch.bfloat16)
    add(fused, 8, 192, False, torch.float32)
    for row0 in range(0, 200, 10):                                      # 23 bf16 -> bf16 jobs: 2 launches
        add(fused, row0, 10, True, torch.bfloat16)
    for i, s in enumerate(srcs):
        for tr in (False, True):
            for out_dt in (torch.float32, torch.bfloat16):
                add(s, i % 3, s.shape[0] - i % 3, tr, out_dt, pad=8 if (i + tr) % 2 else 0)
    assert len(jobs) > 16
    print(f"convert_matrices {len(jobs)} jobs", flush=True)
    mi.convert_matrices(jobs)
    for k, (dst, w, pad) in enumerate(want):
        if pad:
            tr_view = dst[:, :dst.shape[1] - pad]
            assert torch.equal(tr_view, w), k
            assert torch.all(dst[:, dst.shape[1] - pad:] == 7.0), k
        else:
            assert torch.equal(dst, w), k


def test_convert_matrices_overlap_runs_nothing(mi, dev):
    """Two destinations that overlap: the call fails and writes nothing."""
    import torch

    src = torch.randn((64, 64), device=dev).to(torch.bfloat16)
    out = torch.full((96, 64), 7.0, dtype=torch.bfloat16, device=dev)
    jobs = [(src, mi.MI_BF16, 64, 0, 64, 64, True, out[:64]), (src, mi.MI_BF16, 64, 0, 64, 64, False, out[32:])]
    with pytest.raises(mi.MiError) as e:
        mi.convert_matrices(jobs)
    assert e.value.code == 5 and "job" in str(e.value)
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)


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
