"""bench.py's HBM-traffic evidence (no GPU): the summary made from two rocprofv3 --pmc runs
(FETCH_SIZE, WRITE_SIZE) carries the hash of the kernel sources it was measured on, and
bench.py reports `roofline.traffic` from it only while this tree's sources hash the same.

The table generator is checked on synthetic counter files whose values are known: every
dispatch of a GEMM reads a counter value that encodes its position in the launch order, so
a misaligned launch order or a wrong calibration factor shows up in the averages.
"""
import csv
import os
import shutil
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    sys.path.insert(0, ROOT)
    import bench as b

    return b


def _write_counters(d, counter, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for i, (name, v) in enumerate(rows):
            w.writerow([i + 1, name, counter, v])


def test_stale_summary_is_refused(bench, tmp_path, monkeypatch):
    good = tmp_path / "good.md"
    good.write_text(f"kernel sources sha16: `{bench.sources_sha16('block')}`\n\n"
                    "| key | kernels | launches | F | W | bytes | alg | ratio |\n"
                    "| dlds bf16 256x256 NT split1 | k | 5 | 1 | 2 | 123456 | 100 | 1.2 |\n")
    monkeypatch.setitem(bench.TRAFFIC_FILES, "block", str(good))
    assert bench.hbm_bytes_per_launch("dlds bf16 256x256 NT split1", "block") == (123456, None)
    val, note = bench.hbm_bytes_per_launch("dlds bf16 256x192 NN split1", "block")
    assert val is None and "no row" in note
    stale = tmp_path / "stale.md"
    stale.write_text(good.read_text().replace(bench.sources_sha16("block"), "0123456789abcdef"))
    monkeypatch.setitem(bench.TRAFFIC_FILES, "block", str(stale))
    val, note = bench.hbm_bytes_per_launch("dlds bf16 256x256 NT split1", "block")
    assert val is None and "stale" in note
    monkeypatch.setitem(bench.TRAFFIC_FILES, "block", str(tmp_path / "missing.md"))
    assert bench.hbm_bytes_per_launch("dlds bf16 256x256 NT split1", "block")[0] is None


def test_source_hash_follows_the_kernel_sources(bench, tmp_path, monkeypatch):
    """A byte changed in one kernel source changes the hash (so an old summary goes stale)."""
    h0 = bench.sources_sha16("block")
    src = os.path.join(ROOT, bench.KERNEL_SOURCES["block"][0])
    copy = tmp_path / "root"
    rel = bench.KERNEL_SOURCES["block"]
    for r in rel:
        os.makedirs(copy / os.path.dirname(r), exist_ok=True)
        shutil.copy(os.path.join(ROOT, r), copy / r)
    monkeypatch.setattr(bench, "ROOT", str(copy))
    assert bench.sources_sha16("block") == h0
    with open(copy / rel[0], "ab") as f:
        f.write(b" ")
    assert bench.sources_sha16("block") != h0
    assert os.path.exists(src)


def test_traffic_table_block(bench, tmp_path, capsys):
    """Synthetic counters for the configuration-3 block run (--steps 2 --warmup 1: 7 steps of
    15 GEMM launches), a 1 GiB copy reading FETCH 2^19 KiB and WRITE 2^20 KiB (factors 2, 1).
    GEMM i of the step order reads FETCH = i + 1 and WRITE = 10 * (i + 1) KiB in every step."""
    pytest.importorskip("numpy")
    seq, _ = bench.block_sequence(False, "reference")
    assert all(" split1 " in s[4] + " " for s in seq)  # configuration 3 plans no split-K
    n_steps = 1 + 1 + 3 + 2
    fetch, write = [("torch_setup_kernel", 5.0)], [("torch_setup_kernel", 5.0)]
    for _ in range(n_steps):
        for i, s in enumerate(seq):
            fetch.append(("void mig::gemm_dlds_kernel<...>(mig::Params)", float(i + 1)))
            write.append(("void mig::gemm_dlds_kernel<...>(mig::Params)", float(10 * (i + 1))))
    fetch.append(("__amd_rocclr_copyBuffer", float(1 << 19)))
    write.append(("__amd_rocclr_copyBuffer", float(1 << 20)))
    fd, wd = str(tmp_path / "f"), str(tmp_path / "w")
    _write_counters(fd, "FETCH_SIZE", fetch)
    _write_counters(wd, "WRITE_SIZE", write)
    sys_argv = sys.argv
    try:
        sys.argv = ["bench.py", "--workload", "block", "--steps", "2", "--warmup", "1",
                    "--traffic-table", fd, wd]
        args = bench.parse()
    finally:
        sys.argv = sys_argv
    bench.traffic_table_main(args)
    out = capsys.readouterr().out
    assert f"kernel sources sha16: `{bench.sources_sha16('block')}`" in out
    rows = {}
    for line in out.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 8 and cells[2].isdigit():
            rows[cells[0]] = cells
    for i, s in enumerate(seq):
        key = f"{s[0]} {s[2]}"
        c = rows[key]
        assert int(c[2]) == n_steps
        # FETCH scaled x2, WRITE x1; bytes = (F + W) KiB * 1024
        assert float(c[3]) == pytest.approx(2 * (i + 1))
        assert float(c[4]) == pytest.approx(10 * (i + 1))
        assert int(c[5]) == (2 * (i + 1) + 10 * (i + 1)) * 1024
    # a description row averages its GEMMs' launches
    for desc in {s[4].rsplit(" tiles", 1)[0] for s in seq}:
        idx = [i for i, s in enumerate(seq) if s[4].rsplit(" tiles", 1)[0] == desc]
        want = sum(12 * (i + 1) for i in idx) / len(idx) * 1024
        assert int(rows[desc][5]) == pytest.approx(want, abs=1024)


def test_traffic_table_rejects_misaligned_runs(bench, tmp_path):
    fd, wd = str(tmp_path / "f"), str(tmp_path / "w")
    rows = [("void mig::gemm_dlds_kernel<...>(mig::Params)", 1.0)] * 7 + \
        [("__amd_rocclr_copyBuffer", float(1 << 19))]
    _write_counters(fd, "FETCH_SIZE", rows)
    _write_counters(wd, "WRITE_SIZE", rows)
    sys_argv = sys.argv
    try:
        sys.argv = ["bench.py", "--workload", "block", "--steps", "2", "--warmup", "1",
                    "--traffic-table", fd, wd]
        args = bench.parse()
    finally:
        sys.argv = sys_argv
    with pytest.raises(SystemExit):
        bench.traffic_table_main(args)


def test_traffic_table_per_kernel(bench, tmp_path, capsys):
    """The per-kernel summary of the norm workload: each kernel averaged over its launches
    (template arguments dropped), and one backward call's row summing its two kernels."""
    fetch, write = [], []
    for i in range(3):
        fetch += [("void mig::(anonymous namespace)::norm_fwd_vec<true, false, 4>(mig::NormParams)", 100.0 + i),
                  ("void mig::(anonymous namespace)::norm_bwd_vec<true, false, 4, true>(mig::NormParams)", 200.0),
                  ("void mig::(anonymous namespace)::norm_dw_reduce<false>(mig::NormParams)", 10.0)]
        write += [("x", 50.0), ("x", 60.0), ("x", 1.0)]
    fetch.append(("__amd_rocclr_copyBuffer", float(1 << 20)))
    write.append(("__amd_rocclr_copyBuffer", float(1 << 20)))
    write = [(f[0], w[1]) for f, w in zip(fetch, write)]
    fd, wd = str(tmp_path / "f"), str(tmp_path / "w")
    _write_counters(fd, "FETCH_SIZE", fetch)
    _write_counters(wd, "WRITE_SIZE", write)
    sys_argv = sys.argv
    try:
        sys.argv = ["bench.py", "--workload", "norm", "--steps", "2", "--warmup", "1",
                    "--traffic-table", fd, wd]
        args = bench.parse()
    finally:
        sys.argv = sys_argv
    bench.traffic_table_main(args)
    out = capsys.readouterr().out
    rows = {}
    for line in out.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 8 and cells[2].isdigit():
            rows[cells[0]] = cells
    assert int(rows["norm_fwd_vec"][2]) == 3
    assert int(rows["norm_fwd_vec"][5]) == int(round((101.0 + 50.0) * 1024))  # mean FETCH 101
    assert int(rows[bench.NORM_BWD_KEY][5]) == (210 + 61) * 1024
    assert bench.NORM_BWD_KEY in out and "norm_dw_reduce" in rows
