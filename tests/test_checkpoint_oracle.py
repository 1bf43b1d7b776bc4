"""The checkpoint restatement in the oracle (checkpoint_weights, Checkpoint.cpp:28-83,
390-570) against the safetensors library's own reading of the same files (plus torch
slicing and transposes), and the C++ header reader (mi_bridge::SafetensorsFile, run by
tests/cpp/test_safetensors without a GPU) against Python's json on valid and malformed
files."""
import json
import os
import struct
import subprocess

import numpy as np
import pytest

from checkpoint_files import CFG, expected_engine, write_engine_file, write_python_file

HERE = os.path.dirname(os.path.abspath(__file__))
READER = os.path.join(HERE, "cpp", "test_safetensors")


def test_python_format_against_library(oracle, tmp_path):
    path = str(tmp_path / "mlx.safetensors")
    tensors = write_python_file(path)
    got = oracle.checkpoint_weights(path, CFG)
    want = expected_engine(tensors)
    assert set(got) == set(want)
    for k in want:
        assert got[k].shape == want[k].shape and np.array_equal(got[k], want[k]), k


def test_engine_format_against_library(oracle, tmp_path):
    import torch

    for dt in (torch.float32, torch.bfloat16):
        path = str(tmp_path / f"engine_{str(dt)[6:]}.safetensors")
        tensors = write_engine_file(path, dtype=dt)
        got = oracle.checkpoint_weights(path, CFG)
        for k, v in tensors.items():
            assert np.array_equal(got[k], v.float().numpy()), k


def _write_raw(path, header: bytes, payload: bytes = b"", declared=None):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header) if declared is None else declared))
        f.write(header)
        f.write(payload)


def _run_reader(paths):
    assert os.path.exists(READER), "tests/cpp/test_safetensors not built (run __graft_entry__.build())"
    out = subprocess.run([READER] + paths, capture_output=True, text=True, check=True, timeout=60)
    return out.stdout.strip().split("\n")


def test_cpp_header_reader(tmp_path):
    paths = []
    # 1: a library-written file
    p1 = str(tmp_path / "lib.safetensors")
    write_python_file(p1)
    paths.append(p1)
    # 2: names that are prefixes / substrings of each other, escapes, metadata, padding
    head = {"__metadata__": {"k": "v \\\" {"}, "a": {"dtype": "F32", "shape": [2], "data_offsets": [8, 16]},
            "ab": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
            "x\"yé": {"dtype": "BF16", "shape": [1, 2], "data_offsets": [16, 20]}}
    h = json.dumps(head).encode() + b"   "
    p2 = str(tmp_path / "names.safetensors")
    _write_raw(p2, h, bytes(20))
    paths.append(p2)
    # 3..7: malformed files
    bad = {
        "short": lambda p: open(p, "wb").write(b"\x01\x02"),
        "biglen": lambda p: _write_raw(p, b"{}", declared=(11 << 20)),
        "offsets": lambda p: _write_raw(p, json.dumps({"t": {"dtype": "F32", "shape": [4],
                                                              "data_offsets": [0, 16]}}).encode(), bytes(8)),
        "sizes": lambda p: _write_raw(p, json.dumps({"t": {"dtype": "F32", "shape": [3],
                                                            "data_offsets": [0, 16]}}).encode(), bytes(16)),
        "json": lambda p: _write_raw(p, b'{"t": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]', bytes(4)),
    }
    for k, fn in bad.items():
        p = str(tmp_path / f"bad_{k}.safetensors")
        fn(p)
        paths.append(p)
    lines = _run_reader(paths)
    assert len(lines) == len(paths)
    # file 1: every tensor with Python's view of the header
    with open(p1, "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
        h1 = json.loads(f.read(n))
    toks = lines[0].split()
    assert toks[0] == "OK" and int(toks[1]) == len(h1) - 1 and toks[2] == "python=1"
    seen = {}
    for t in toks[3:]:
        name, dt, shape, rng = t.split(":")
        seen[name] = (dt, shape, rng)
    for name, ent in h1.items():
        if name == "__metadata__":
            continue
        b, e = ent["data_offsets"]
        assert seen[name] == (ent["dtype"], "x".join(map(str, ent["shape"])), f"{b}-{e}"), name
    # file 2: the exact entries, the escaped name decoded
    assert lines[1].startswith("OK 3 python=0")
    assert " a:F32:2:8-16" in lines[1] and " ab:F32:2:0-8" in lines[1]
    assert ' x"yé:BF16:1x2:16-20' in lines[1]
    for line in lines[2:]:
        assert line.startswith("ERR "), line
