"""Seeded sweep of the checkpoint conversion (mi_convert_matrices; the reference loader's
widening, [out, in] -> [in, out] transposes and wqkv / w12 de-fusion, Checkpoint.cpp:28-83,
404-570): random jobs of every source dtype (f32, bf16, f16) into f32 or bf16, transposed or
not, with source rows padded past the columns taken (src_ld > cols), row ranges that start
and end anywhere, column counts on and off whole 16-byte vectors, and padded destinations,
several jobs per call.  Conversions are exact (widening) or round to nearest even (to bf16),
as torch converts: every element must match bit for bit, and the destination's pad columns
must keep their values.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _jobs(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        cols = int(rng.choice([int(rng.integers(1, 200)), 8 * int(rng.integers(1, 90))]))
        src_ld = cols + int(rng.choice([0, 0, int(rng.integers(1, 17)), 8 * int(rng.integers(1, 9))]))
        R = int(rng.integers(1, 700))
        row0 = int(rng.integers(0, R))
        rows = int(rng.integers(1, R - row0 + 1))
        out.append(dict(R=R, src_ld=src_ld, cols=cols, row0=row0, rows=rows,
                        src=str(rng.choice(["f32", "bf16", "f16"])), dst=str(rng.choice(["f32", "bf16"])),
                        tr=bool(rng.integers(0, 2)), pad=int(rng.choice([0, 0, 3, 8]))))
    return out


@pytest.mark.parametrize("part", range(4))
def test_convert_matrices_sweep(mi, dev, part):
    import torch

    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
    code = {"f32": mi.MI_F32, "bf16": mi.MI_BF16, "f16": mi.MI_F16}
    g = torch.Generator(device=dev)
    g.manual_seed(8400 + part)
    specs = _jobs(8400 + part, 10)
    jobs, checks = [], []
    for j in specs:
        print(f"convert sweep {j}", flush=True)
        src = torch.randn((j["R"], j["src_ld"]), generator=g, device=dev).to(tdt[j["src"]])
        drows, dcols = (j["cols"], j["rows"]) if j["tr"] else (j["rows"], j["cols"])
        dst = torch.full((drows, dcols + j["pad"]), 7.0, dtype=tdt[j["dst"]], device=dev)
        jobs.append((src, code[j["src"]], j["src_ld"], j["row0"], j["rows"], j["cols"], j["tr"],
                     dst[:, :dcols]))
        w = src[j["row0"]:j["row0"] + j["rows"], :j["cols"]].float()
        checks.append((dst, (w.t() if j["tr"] else w).to(tdt[j["dst"]]), dcols))
    mi.convert_matrices(jobs)
    for k, (dst, want, dcols) in enumerate(checks):
        assert torch.equal(dst[:, :dcols], want), f"job {k}: {specs[k]}"
        assert torch.all(dst[:, dcols:] == 7.0), f"job {k} pad columns"
