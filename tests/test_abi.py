"""CPU-side tests of the C-ABI library: it loads, exports every declared symbol,
and validates arguments (status codes and messages) without touching a GPU.
Also the host-side shape rules of the Tensor::matmul mirror (Tensor.cpp:174-209)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_c_functions():
    text = open(os.path.join(ROOT, "include", "mi_gemm.h")).read()
    return sorted(set(re.findall(r"\b(mi_[a-z_0-9]+)\s*\(", text)))


def test_header_symbols_exported(mi):
    names = _declared_c_functions()
    assert len(names) >= 10
    lib = mi.load_library()
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(mi.C_SYMBOLS)


def test_cpp_bridge_symbols_exported(mi):
    out = subprocess.run(["nm", "-DC", "--defined-only", mi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    hdr = open(os.path.join(ROOT, "include", "gemm_bridge.hpp")).read()
    decl = set(re.findall(r"^(?:void|bool|int|void\*|std::vector<size_t>)\s+([a-z_0-9]+)\(",
                          hdr, flags=re.M))
    assert {"gemm_bf16", "gemm_backward", "gemm_proj_trans_b", "gemm_proj", "gemm_ffn",
            "fused_swiglu_gemm", "residual_add", "matmul"} <= decl
    for n in decl:
        assert f"mi_bridge::{n}(" in out, n


def test_version(mi):
    assert "gfx950" in mi.version()


def _call(mi, M=64, N=64, K=64, lda=None, ldb=None, ldc=None, A=16, B=32, C=48, dt_in=1, dt_c=1,
          transA=0, transB=0, epi=None):
    lib = mi.load_library()
    lda = lda if lda is not None else (M if transA else K)
    ldb = ldb if ldb is not None else (K if transB else N)
    ldc = ldc if ldc is not None else N
    st = lib.mi_gemm(None, transA, transB, M, N, K, 1.0, ctypes.c_void_p(A), lda,
                     ctypes.c_void_p(B), ldb, dt_in, 0.0, ctypes.c_void_p(C), ldc, dt_c,
                     epi, None, 0)
    return st, lib.mi_last_error().decode()


def test_validation_status_codes(mi):
    # Arguments are rejected before any device work, so these run without a GPU.
    assert _call(mi, M=-1)[0] == 1                         # MI_ERR_SHAPE
    st, msg = _call(mi, lda=10)
    assert st == 2 and "lda" in msg                        # MI_ERR_LD
    assert _call(mi, transA=1, lda=32)[0] == 2
    assert _call(mi, ldb=3, transB=1)[0] == 2
    assert _call(mi, ldc=8)[0] == 2
    assert _call(mi, A=0)[0] == 3                          # MI_ERR_NULL
    assert _call(mi, C=0)[0] == 3
    assert _call(mi, dt_in=7)[0] == 4                      # MI_ERR_DTYPE
    assert _call(mi, dt_c=9)[0] == 4
    e = mi.MiEpilogue()
    e.A2, e.B2 = 64, 128
    assert _call(mi, epi=ctypes.byref(e))[0] == 5          # MI_ERR_UNSUPPORTED
    e2 = mi.MiEpilogue()
    e2.A2 = 64
    assert _call(mi, epi=ctypes.byref(e2), transA=1, lda=64)[0] == 5
    # empty outputs are a successful no-op (MetalBridge.mm:622-623,693)
    assert _call(mi, M=0, A=0, B=0, C=0)[0] == 0
    assert _call(mi, N=0, A=0, B=0, C=0)[0] == 0


def test_batch_validation(mi):
    lib = mi.load_library()
    bt = mi.make_batch(0)
    st = lib.mi_gemm_batched(None, 0, 0, 8, 8, 8, 1.0, ctypes.c_void_p(16), 8,
                             ctypes.c_void_p(16), 8, 1, 0.0, ctypes.c_void_p(16), 8, 1,
                             ctypes.byref(bt), None, None, 0)
    assert st == 1
    bt = mi.make_batch(4, heads=2, causal=9)
    st = lib.mi_gemm_batched(None, 0, 0, 8, 8, 8, 1.0, ctypes.c_void_p(16), 8,
                             ctypes.c_void_p(16), 8, 1, 0.0, ctypes.c_void_p(16), 8, 1,
                             ctypes.byref(bt), None, None, 0)
    assert st == 1 and "causal" in lib.mi_last_error().decode()
    st = lib.mi_gemm_batched(None, 0, 0, 8, 8, 8, 1.0, None, 8, None, 8, 1, 0.0, None, 8, 1,
                             None, None, None, 0)
    assert st == 3


def test_no_device_reports_status(mi):
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    assert mi.load_library().mi_init() == 8                 # MI_ERR_NO_DEVICE
    assert "gfx950" in mi.load_library().mi_last_error().decode()


def test_aux_validation(mi):
    lib = mi.load_library()
    assert lib.mi_residual_add(None, None, None, 0, 1) == 0
    assert lib.mi_residual_add(None, None, None, 5, 1) == 3
    assert lib.mi_residual_add(None, ctypes.c_void_p(16), ctypes.c_void_p(16), 5, 3) == 4
    assert lib.mi_softmax_causal(None, ctypes.c_void_p(16), 4, 8, 4, 1) == 2
    assert lib.mi_softmax_bwd(None, None, None, 4, 8, 8, 1.0, 1) == 3
    p16 = ctypes.c_void_p(16)
    fa = lib.mi_flash_attn_fwd
    assert fa(None, None, None, None, None, None, 0, 4, 2, 64, 128, 1, 1) == 0   # empty batch
    assert fa(None, None, p16, p16, p16, None, 1, 4, 2, 64, 128, 1, 1) == 3      # Q NULL
    assert fa(None, p16, p16, p16, p16, None, 1, 4, 3, 64, 128, 1, 1) == 1       # 4 % 3 heads
    assert fa(None, p16, p16, p16, p16, None, 1, 4, 2, 64, 96, 1, 1) == 5        # head_dim 96
    assert fa(None, p16, p16, p16, p16, None, 1, 4, 2, 64, 128, 1, 7) == 1       # layout
    assert fa(None, ctypes.c_void_p(18), p16, p16, p16, None, 1, 4, 2, 64, 128, 1, 1) == 5
    fb = lib.mi_flash_attn_bwd
    assert fb(None, *([None] * 10), 0, 4, 2, 64, 128, 1, 1, None, 0) == 0        # empty batch
    assert fb(None, *([p16] * 9), None, 1, 4, 2, 64, 128, 1, 1, None, 0) == 3    # delta NULL
    assert fb(None, *([p16] * 10), 1, 4, 2, 64, 96, 1, 1, None, 0) == 5          # head_dim 96
    # dS^T (bf16), then the fp32 partials of the balanced dK/dV units (128 floats per row)
    assert lib.mi_flash_attn_bwd_workspace_size(8, 16, 1024) == 8 * 16 * 1024 * (1024 * 2 + 512)
    assert lib.mi_flash_attn_bwd_workspace_size(1, 4, 300) == 0                   # T % 8 != 0
    assert lib.mi_flash_attn_bwd_workspace_size(1, 1, 32768) == 0                 # T > 32767
    assert lib.mi_flash_attn_bwd_workspace_size(1, 1, 32760) == 32760 * (32760 * 2 + 512)


def test_convert_matrices_validation(mi):
    """mi_convert_matrices checks every job before anything runs (no device needed):
    the job count, each job's arguments (the message names the job), and that no
    destination overlaps another job's source or destination; sources may share bytes."""
    lib = mi.load_library()

    def job(src, dst, row0=0, rows=64, cols=64, tr=1, sdt=mi.MI_BF16, ddt=mi.MI_BF16, ld=64):
        j = mi.MiConvertJob()
        j.src, j.src_dtype, j.transpose, j.src_ld = src, sdt, tr, cols
        j.row0, j.rows, j.cols = row0, rows, cols
        j.dst, j.dst_dtype, j.reserved, j.dst_ld = dst, ddt, 0, ld
        return j

    def run(*jobs):
        arr = (mi.MiConvertJob * len(jobs))(*jobs)
        return lib.mi_convert_matrices(None, arr, len(jobs)), lib.mi_last_error().decode()

    S, D = 1 << 20, 1 << 24            # fake device addresses: no call reaches the GPU
    assert lib.mi_convert_matrices(None, None, 0) == 0
    assert lib.mi_convert_matrices(None, None, -1) == 1
    assert lib.mi_convert_matrices(None, None, 2) == 3
    assert run(job(S, D, rows=0))[0] == 0                       # empty jobs only: nothing to do
    st, msg = run(job(S, D), job(S, D + 8192, sdt=7))
    assert st == 4 and "job 1" in msg                            # dtype of the second job
    st, msg = run(job(S, D), job(S, D + 8192, ld=32))
    assert st == 2 and "job 1" in msg                            # dst_ld < rows
    st, msg = run(job(S, D), job(S, D + 4096))                   # destinations 8 KiB each
    assert st == 5 and "job 1" in msg and "job 0" in msg
    st, msg = run(job(S, D), job(D + 100, D + 65536))            # a source inside job 0's dst
    assert st == 5 and "job 1" in msg
    st, msg = run(job(S, D), job(S + 64, D - 8192 + 2))          # dst runs into job 0's dst
    assert st == 5
    bad = job(S, D + 8192)
    bad.reserved = 1
    st, msg = run(job(S, D), bad)
    assert st == 1 and "job 1" in msg and "reserved" in msg      # MI_ERR_SHAPE
    # row ranges of one fused source (disjoint destinations) pass validation: without a
    # GPU the call then stops at device initialisation.  With a GPU visible it would launch
    # the conversion on the fake addresses, so it is left out there.
    import torch

    if not torch.cuda.is_available():
        st, _ = run(job(S, D, row0=0, rows=64), job(S, D + 8192, row0=32, rows=64))
        assert st == 8                                           # MI_ERR_NO_DEVICE


def test_convert_job_layout(mi):
    """The ctypes mirror of mi_convert_job has the C struct's size and field offsets
    (pointers and int64 fields 8-aligned, the int32 pairs packed)."""
    J = mi.MiConvertJob
    assert ctypes.sizeof(J) == 72
    want = {"src": 0, "src_dtype": 8, "transpose": 12, "src_ld": 16, "row0": 24, "rows": 32,
            "cols": 40, "dst": 48, "dst_dtype": 56, "reserved": 60, "dst_ld": 64}
    assert {n: getattr(J, n).offset for n in want} == want
    hdr = open(os.path.join(ROOT, "include", "mi_gemm.h")).read()
    body = hdr[hdr.index("typedef struct mi_convert_job"):hdr.index("} mi_convert_job;")]
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    order = re.findall(r"\b(src|src_dtype|transpose|src_ld|row0|rows|cols|dst|dst_dtype|reserved|dst_ld)\b", body)
    assert order == list(want), order


def test_matmul_shape_rules(mi):
    assert mi.matmul_shape((2, 3), (3, 2)) == (2, 2)
    assert mi.matmul_shape((8, 1024, 2048), (2048, 3072)) == (8, 1024, 3072)
    assert mi.matmul_shape((8, 16, 1024, 128), (8, 16, 128, 1024)) == (8, 16, 1024, 1024)
    cases = [((3,), (3, 2), "Matmul requires at least 2 dimensions"),
             ((2, 2, 3), (4, 2), "Inner dimensions must match for projection"),
             ((2, 2, 3), (3, 3, 2), "Batch dimension must match for matmul"),
             ((2, 2, 3), (2, 4, 2), "Inner dimensions must match for matmul"),
             ((1, 2, 2, 3), (3, 3, 2), "Batch size must match for matrix multiplication"),
             ((2, 3), (4, 2), "Inner dimensions must match for matmul")]
    for a, b, msg in cases:
        with pytest.raises(ValueError, match=msg):
            mi.matmul_shape(a, b)


def test_workspace_query(mi):
    # few output tiles and a very long K: split-K space is requested
    assert mi.workspace_size(1, 0, 1024, 1024, 65536) > 0
    assert mi.workspace_size(0, 0, 8192, 5632, 2048) == 0
    assert mi.workspace_size(0, 0, 0, 5, 5) == 0
    # a small output with a long K splits even where 256x256 tiles would sit mostly empty
    assert "split8" in mi.describe(1, 0, 100, 60, 70000, workspace_bytes=64 << 20)


def _planned_split(mi, *args, **kw):
    text = mi.describe(*args, **kw)
    m = re.search(r"split(\d+)", text)
    assert m, text
    return int(m.group(1))


def test_split_plans_fit_the_workspace(mi):
    """Planner invariant behind the MI_ERR_WORKSPACE guard in run(): a split-K plan
    never writes more partials than the workspace holds, splits * M * N * batch * 4
    <= workspace bytes, for every shape, dtype and workspace size; and the size
    mi_gemm_workspace_size reports is exactly what its plan writes. Planner only:
    no device, no kernel."""
    shapes = [(100, 60, 70000, 1), (512, 768, 768, 1), (768, 768, 2048, 1), (2048, 768, 768, 1),
              (1024, 1024, 65536, 1), (256, 384, 30000, 1), (2048, 2048, 8192, 1),
              (8192, 32000, 2048, 1), (128, 128, 4096, 3), (64, 4096, 9000, 2), (1, 1, 100000, 1),
              (300, 20, 513, 1), (2048, 5632, 8192, 1), (96, 96, 1 << 20, 1)]
    seen_split = 0
    for dt in (mi.MI_BF16, mi.MI_F32):
        for M, N, K, batch in shapes:
            full = mi.workspace_size(1, 0, M, N, K, dt, mi.MI_F32, batch)
            sp_full = _planned_split(mi, 1, 0, M, N, K, dt, batch, 0, full)
            assert full == (sp_full * M * N * batch * 4 if sp_full > 1 else 0), (M, N, K, dt)
            for ws in sorted({0, 4, full // 2, full - 4 if full else 0, full, full * 3,
                              M * N * batch * 4 * 2 - 4, M * N * batch * 4 * 2, 64 << 20, 1 << 34}):
                if ws < 0:
                    continue
                sp = _planned_split(mi, 1, 0, M, N, K, dt, batch, 0, ws)
                assert sp == 1 or sp * M * N * batch * 4 <= ws, (M, N, K, dt, batch, ws, sp)
                assert sp <= max(sp_full, 1), (M, N, K, dt, ws)
                seen_split = max(seen_split, sp)
    assert seen_split >= 3


def test_block_plans(mi):
    """The planner's picks for the benchmark configurations' GEMM sets (describe only, no
    device): configuration 3's bf16 set (256x192 for the qkv forward and the large weight
    gradients, wave-level split-K tiles for the o / qkv weight gradients, 256x256 elsewhere;
    no split), and configuration 2's fp32 set on the direct-to-LDS tiles with the
    workspace the bench passes (64x64 where a split of 2 or 3, or a 64x64 round, balances
    the CUs best; 64x128 for the short-K outputs of 192 and 512 tiles)."""
    ws = 512 << 20
    want3 = {  # (M, N, K, tA, tB): description prefix
        (8192, 3072, 2048, 0, 0): "dlds bf16 256x192 NN split1",
        (8192, 2048, 2048, 0, 0): "dlds bf16 256x256 NN split1",
        (8192, 5632, 2048, 0, 0): "dlds bf16 256x256 NN split1",
        (8192, 2048, 5632, 0, 0): "dlds bf16 256x256 NN split1",
        (5632, 2048, 8192, 1, 0): "dlds bf16 256x192 TN split1",
        (8192, 5632, 2048, 0, 1): "dlds bf16 256x256 NT split1",
        (2048, 5632, 8192, 1, 0): "dlds bf16 256x192 TN split1",
        (8192, 2048, 5632, 0, 1): "dlds bf16 256x256 NT split1",
        (2048, 2048, 8192, 1, 0): "dlds-kg2 bf16 128x128 TN split1",
        (8192, 2048, 2048, 0, 1): "dlds bf16 256x256 NT split1",
        (2048, 3072, 8192, 1, 0): "dlds-kg2 bf16 128x192 TN split1",
        (8192, 2048, 3072, 0, 1): "dlds bf16 256x256 NT split1",
    }
    for (M, N, K, tA, tB), w in want3.items():
        assert mi.describe(tA, tB, M, N, K, mi.MI_BF16, workspace_bytes=ws).startswith(w), (M, N, K, tA, tB)
    want2 = {
        (2048, 2304, 768, 0, 0): "dlds f32 64x64 NN split1",
        (2048, 768, 2304, 0, 1): "dlds f32 64x64 NT split2",
        (768, 2304, 2048, 1, 0): "dlds f32 64x64 TN split1",
        (2048, 768, 768, 0, 0): "dlds f32 64x128 NN split1",
        (2048, 768, 768, 0, 1): "dlds f32 64x128 NT split1",
        (768, 768, 2048, 1, 0): "dlds f32 64x64 TN split3",
        (2048, 2048, 768, 0, 0): "dlds f32 64x128 NN split1",
        (2048, 768, 2048, 0, 1): "dlds f32 64x64 NT split2",
        (768, 2048, 2048, 1, 0): "dlds f32 64x64 TN split2",
        (2048, 768, 2048, 0, 0): "dlds f32 64x64 NN split2",
        (2048, 2048, 768, 0, 1): "dlds f32 64x128 NT split1",
        (2048, 768, 2048, 1, 0): "dlds f32 64x64 TN split2",
        (512, 768, 768, 0, 1): "dlds f32 64x128 NT split5",   # configuration 1
    }
    for (M, N, K, tA, tB), w in want2.items():
        assert mi.describe(tA, tB, M, N, K, mi.MI_F32, workspace_bytes=ws).startswith(w), (M, N, K, tA, tB)
    # unaligned fp32 operands (odd K) take the register-staged 128x128 tiles
    assert mi.describe(0, 0, 1000, 600, 333, mi.MI_F32).startswith("regstage f32 128x128")


def test_cross_entropy_validation(mi):
    # mi_cross_entropy rejects bad arguments before any device work.
    lib = mi.load_library()
    vp = ctypes.c_void_p

    def ce(rows=4, vocab=64, ld=64, L=4096, T=8192, RL=12288, LO=16384, G=None, gdt=0, ldg=64, dt=1):
        st = lib.mi_cross_entropy(None, vp(L) if L else None, dt, ld, vp(T) if T else None, rows,
                                  vocab, 0.25, vp(RL) if RL else None, vp(LO) if LO else None,
                                  vp(G) if G else None, gdt, ldg)
        return st, lib.mi_last_error().decode()

    assert ce(rows=0)[0] == 0 and ce(vocab=0)[0] == 0    # no-op, as the reference
    assert ce(rows=-1)[0] == 1                           # MI_ERR_SHAPE
    st, msg = ce(ld=10)
    assert st == 2 and "ld_logits" in msg                # MI_ERR_LD
    st, msg = ce(G=65536, ldg=10)
    assert st == 2 and "ld_grad" in msg
    assert ce(L=0)[0] == 3 and ce(T=0)[0] == 3 and ce(RL=0)[0] == 3   # MI_ERR_NULL
    assert ce(dt=7)[0] == 4                              # MI_ERR_DTYPE
    assert ce(G=65536, gdt=9)[0] == 4
    # a gradient that overlaps the logits without being the same array
    st, msg = ce(G=4096 + 64, gdt=1, ldg=64)
    assert st == 5 and "overlaps" in msg                 # MI_ERR_UNSUPPORTED
    st, msg = ce(L=4097)
    assert st == 5 and "aligned" in msg


def test_lm_head_xent_validation(mi):
    """mi_lm_head_xent's workspace size and argument checks (no device needed)."""
    lib = mi.load_library()
    vp = ctypes.c_void_p
    a256 = lambda b: (b + 255) // 256 * 256  # noqa: E731
    ws = lib.mi_lm_head_xent_workspace_size
    # bf16 logits chunk (rows x chunk rounded up to 8, + 128 when a multiple of 1024), 3 fp32
    # row arrays, fp32 dX accumulator
    assert ws(8192, 2048, 32000, 8192, mi.MI_BF16) == \
        256 + a256(8192 * 8320 * 2) + 3 * a256(8192 * 4) + a256(8192 * 2048 * 4)
    assert ws(100, 64, 777, 100, mi.MI_F32) == 256 + a256(100 * 104 * 2) + 3 * a256(400)
    assert ws(100, 64, 777, 0, mi.MI_F32) == ws(100, 64, 777, 5000, mi.MI_F32) == \
        256 + a256(100 * 784 * 2) + 3 * a256(400)                   # one chunk of the vocab
    assert ws(0, 64, 777, 100, mi.MI_F32) == 0

    def call(rows=4, hidden=64, vocab=100, ldx=64, layout=0, ldw=100, X=4096, W=8192, T=16384,
             RL=20480, dX=None, dxt=1, lddx=64, dW=None, dwt=0, lddw=100, wsb=1 << 20):
        st = lib.mi_lm_head_xent(None, vp(X) if X else None, ldx, vp(W) if W else None, layout, ldw,
                                 vp(T) if T else None, rows, hidden, vocab, 0.25,
                                 vp(RL) if RL else None, None, vp(dX) if dX else None, dxt, lddx,
                                 vp(dW) if dW else None, dwt, lddw, 1.0, 64, vp(1 << 24), wsb)
        return st, lib.mi_last_error().decode()

    assert call(rows=0)[0] == 0 and call(vocab=0)[0] == 0
    assert call(rows=-1)[0] == 1 and call(hidden=0)[0] == 1
    assert call(layout=2)[0] == 5
    assert call(X=0)[0] == 3 and call(W=0)[0] == 3 and call(T=0)[0] == 3 and call(RL=0)[0] == 3
    st, msg = call(ldx=10)
    assert st == 2 and "ldx" in msg
    assert call(ldw=99)[0] == 2                       # layout 0: W [hidden, ldw >= vocab]
    assert call(layout=1, ldw=63)[0] == 2             # layout 1: W [vocab, ldw >= hidden]
    assert call(dX=65536, dxt=7)[0] == 4 and call(dX=65536, lddx=10)[0] == 2
    assert call(dW=65536, dwt=3)[0] == 4 and call(dW=65536, lddw=50)[0] == 2
    assert call(X=4097)[0] == 5
    st, msg = call(wsb=1000)
    assert st == 6 and "workspace" in msg             # MI_ERR_WORKSPACE


def test_rmsnorm_validation(mi):
    # mi_rmsnorm_fwd / _bwd reject bad arguments before any device work.
    lib = mi.load_library()
    vp = ctypes.c_void_p

    def fwd(rows=4, dims=64, ld=64, X=4096, R=None, W=65536, Y=131072, dt=1, wdt=1):
        st = lib.mi_rmsnorm_fwd(None, vp(X) if X else None, vp(R) if R else None,
                                vp(W) if W else None, wdt, vp(Y) if Y else None, None, rows, dims,
                                ld, dt, 1e-5)
        return st, lib.mi_last_error().decode()

    assert fwd(rows=0)[0] == 0 and fwd(dims=0)[0] == 0
    assert fwd(rows=-1)[0] == 1
    st, msg = fwd(ld=10)
    assert st == 2 and "ld" in msg
    assert fwd(X=0)[0] == 3 and fwd(W=0)[0] == 3 and fwd(Y=0)[0] == 3
    assert fwd(dt=5)[0] == 4 and fwd(wdt=5)[0] == 4
    st, msg = fwd(Y=4096 + 64)                      # y overlaps x without being x
    assert st == 5 and "disjoint" in msg
    assert fwd(X=4097)[0] == 5

    def bwd(DY=4096, X=131072, W=65536, DX=262144, DW=None, ws=None, wsb=0, dims=64, rows=4):
        st = lib.mi_rmsnorm_bwd(None, vp(DY) if DY else None, vp(X), vp(W), 1, None,
                                vp(DX) if DX else None, vp(DW) if DW else None, 0, 0.0, rows, dims,
                                dims, 1, 1e-5, vp(ws) if ws else None, wsb)
        return st, lib.mi_last_error().decode()

    need = lib.mi_rmsnorm_bwd_workspace_size(4, 64)
    assert need == 1 * 64 * 4                       # one workgroup for 4 rows
    st, msg = bwd(DW=8192)
    assert st == 6 and "workspace" in msg           # MI_ERR_WORKSPACE
    assert bwd(DW=8192, ws=16384, wsb=need - 4)[0] == 6
    assert bwd(DY=0)[0] == 3 and bwd(DX=0)[0] == 3
    st, msg = bwd(DX=131072 + 2)                    # dx overlaps x without being x
    assert st == 5


def test_profiler_api_without_device(mi):
    """The profiler's C functions on the CPU: nothing is recorded (no call reaches a
    launch without a device), out-of-range records are refused, totals are zero."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    lib = mi.load_library()
    prof = mi.GemmProfiler.instance()
    assert prof is mi.GemmProfiler.instance()
    was = prof.enable()
    assert prof.enable() is True                       # previous state: on
    assert _call(mi)[0] == 8                           # MI_ERR_NO_DEVICE: nothing recorded
    assert lib.mi_profiler_count() == 0 and prof.records() == []
    rec = mi.MiGemmRecord()
    assert lib.mi_profiler_record(0, ctypes.byref(rec)) == 1   # MI_ERR_SHAPE
    assert lib.mi_profiler_record(0, None) == 3                # MI_ERR_NULL
    prof.begin_step()
    mi.reset_profile_stats()
    assert mi.accum_gpu_time_ms() == 0.0 and mi.count_gpu_calls() == 0
    assert prof.enable(was) is True
    assert mi.GemmProfiler.op_name(1, 1, 1, True, False) == "weight gradient (TN)"


def test_noalloc_scratch_bound(mi):
    """mi_gemm_noalloc's static scratch (32 MiB) holds the split-K partials of every
    batch-1 problem on a 256-CU device: a split plan writes at most two 128x128 fp32
    tiles per CU (splits * tiles <= 2 * CUs). Planner only, no device."""
    limit = 32 << 20
    worst = 0
    for dt in (mi.MI_BF16, mi.MI_F32):
        for M in (1, 60, 100, 128, 129, 256, 384, 512, 768, 1000, 1024, 1536, 2048, 4096):
            for N in (1, 64, 200, 256, 384, 768, 1024, 2000, 2048, 5632):
                for K in (4096, 20000, 65536, 1 << 20):
                    for tA, tB in ((0, 0), (1, 0), (0, 1)):
                        worst = max(worst, mi.workspace_size(tA, tB, M, N, K, dt, mi.MI_F32))
    assert 0 < worst <= limit, worst
