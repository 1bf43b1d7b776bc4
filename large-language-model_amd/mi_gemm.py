"""Python mirror of the reference engine's GEMM operator layer, over libmi_gemm.so.

The functions keep the names, argument meaning and error behaviour of the
reference's operator interface:

* ``gemm_bf16 / fused_swiglu_gemm / gemm_ffn / gemm_proj / gemm_backward /
  gemm_proj_trans_b / residual_add / begin_scope / end_scope`` --
  ``metal_bridge::`` (cpp/include/gpu_kernel/MetalBridge.hpp:29-46,78,119-125);
* ``matmul(a, b)`` -- ``Tensor::matmul`` (cpp/src/Tensor.cpp:174-228), raising
  ``ValueError`` (the reference's ``std::invalid_argument``) with the same messages;
* ``attention_forward / attention_backward`` -- the batched GQA products of
  ``Attention::forward/backward`` (cpp/src/Attention.cpp:236-280, 292-348) composed
  from ``gemm_batched`` plus the row softmax kernels.

Tensors are torch CUDA tensors; torch only provides device memory and the current
stream. All arithmetic runs in the HIP kernels of libmi_gemm.so; importing this
module on a machine where the library is missing raises immediately, and there
is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import math
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmi_gemm.so")

MI_F32, MI_BF16, MI_F16 = 0, 1, 2
MI_CAUSAL_NONE, MI_CAUSAL_OUT_LOWER, MI_CAUSAL_A_LOWER, MI_CAUSAL_A_UPPER = 0, 1, 2, 3

# Exported C-ABI symbols (include/mi_gemm.h).
C_SYMBOLS = (
    "mi_init", "mi_last_error", "mi_version", "mi_gemm_workspace_size", "mi_gemm",
    "mi_gemm_batched", "mi_residual_add", "mi_softmax_causal", "mi_softmax_bwd",
    "mi_gemm_describe", "mi_stream_sync", "mi_flash_attn_fwd", "mi_flash_attn_bwd",
    "mi_cross_entropy", "mi_rmsnorm_fwd", "mi_rmsnorm_bwd", "mi_rmsnorm_bwd_workspace_size",
    "mi_convert_matrix", "mi_flash_attn_bwd_workspace_size", "mi_profiler_enable",
    "mi_profiler_begin_step", "mi_profiler_count", "mi_profiler_record", "mi_profiler_totals",
    "mi_profiler_reset", "mi_gemm_noalloc", "mi_flash_attn_fwd_scaled", "mi_flash_attn_bwd_scaled",
    "mi_convert_matrices", "mi_rmsnorm_fold_weight", "mi_lm_head_xent",
    "mi_lm_head_xent_workspace_size",
)
MI_ATTN_O_BHTD, MI_ATTN_O_BTHD = 0, 1


class MiError(RuntimeError):
    """A non-zero mi_status from the C ABI."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn}: status {code}: {msg}")
        self.code = code


class MiEpilogue(ctypes.Structure):
    _fields_ = [
        ("bias", ctypes.c_void_p), ("bias_dtype", ctypes.c_int32),
        ("residual", ctypes.c_void_p), ("residual_dtype", ctypes.c_int32),
        ("ldr", ctypes.c_int64),
        ("B2", ctypes.c_void_p), ("A2", ctypes.c_void_p), ("row_scale", ctypes.c_void_p),
    ]


class MiBatch(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int64), ("heads", ctypes.c_int64),
        ("a_outer", ctypes.c_int64), ("a_inner", ctypes.c_int64), ("a_group", ctypes.c_int64),
        ("b_outer", ctypes.c_int64), ("b_inner", ctypes.c_int64), ("b_group", ctypes.c_int64),
        ("c_outer", ctypes.c_int64), ("c_inner", ctypes.c_int64), ("c_group", ctypes.c_int64),
        ("r_outer", ctypes.c_int64), ("r_inner", ctypes.c_int64),
        ("k_segments", ctypes.c_int64), ("seg_a", ctypes.c_int64), ("seg_b", ctypes.c_int64),
        ("causal", ctypes.c_int32), ("mask_value", ctypes.c_float),
    ]


class MiConvertJob(ctypes.Structure):
    """mi_convert_job: the arguments of one mi_convert_matrix call."""
    _fields_ = [
        ("src", ctypes.c_void_p), ("src_dtype", ctypes.c_int32), ("transpose", ctypes.c_int32),
        ("src_ld", ctypes.c_int64), ("row0", ctypes.c_int64), ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64), ("dst", ctypes.c_void_p), ("dst_dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32), ("dst_ld", ctypes.c_int64),
    ]


class MiGemmRecord(ctypes.Structure):
    _fields_ = [
        ("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
        ("batch", ctypes.c_int64),
        ("transA", ctypes.c_int32), ("transB", ctypes.c_int32),
        ("dtype_in", ctypes.c_int32), ("dtype_c", ctypes.c_int32),
        ("splits", ctypes.c_int32), ("gpu_ms", ctypes.c_double),
        ("kernel", ctypes.c_char * 64),
    ]


_lib = None


def load_library():
    """Load libmi_gemm.so (built by __graft_entry__.build()); raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
    # torch ships its own libamdhip64.so.7.  Loading torch first makes the
    # library's libamdhip64.so.7 dependency resolve to that already-loaded copy;
    # loading the library first would bring a second HIP/HSA runtime into the
    # process, and the two cannot share the device.
    import torch  # noqa: F401

    L = ctypes.CDLL(LIB_PATH)
    vp, i64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float
    L.mi_init.restype = ctypes.c_int
    L.mi_last_error.restype = ctypes.c_char_p
    L.mi_version.restype = ctypes.c_char_p
    L.mi_gemm_workspace_size.restype = ctypes.c_size_t
    L.mi_gemm_workspace_size.argtypes = [ctypes.c_int, ctypes.c_int, i64, i64, i64, i32, i32, i64]
    L.mi_gemm.restype = ctypes.c_int
    L.mi_gemm.argtypes = [vp, ctypes.c_int, ctypes.c_int, i64, i64, i64, f32, vp, i64, vp, i64,
                          i32, f32, vp, i64, i32, ctypes.POINTER(MiEpilogue), vp, ctypes.c_size_t]
    L.mi_gemm_noalloc.restype = ctypes.c_int
    L.mi_gemm_noalloc.argtypes = [vp, ctypes.c_int, ctypes.c_int, i64, i64, i64, f32, vp, i64, vp,
                                  i64, i32, f32, vp, i64, i32, ctypes.POINTER(MiEpilogue)]
    L.mi_gemm_batched.restype = ctypes.c_int
    L.mi_gemm_batched.argtypes = [vp, ctypes.c_int, ctypes.c_int, i64, i64, i64, f32, vp, i64,
                                  vp, i64, i32, f32, vp, i64, i32, ctypes.POINTER(MiBatch),
                                  ctypes.POINTER(MiEpilogue), vp, ctypes.c_size_t]
    L.mi_residual_add.restype = ctypes.c_int
    L.mi_residual_add.argtypes = [vp, vp, vp, i64, i32]
    L.mi_softmax_causal.restype = ctypes.c_int
    L.mi_softmax_causal.argtypes = [vp, vp, i64, i64, i64, i32]
    L.mi_softmax_bwd.restype = ctypes.c_int
    L.mi_softmax_bwd.argtypes = [vp, vp, vp, i64, i64, i64, f32, i32]
    L.mi_gemm_describe.restype = ctypes.c_int
    L.mi_gemm_describe.argtypes = [ctypes.c_int, ctypes.c_int, i64, i64, i64, i32, i64, i32,
                                   ctypes.c_size_t, ctypes.c_char_p, ctypes.c_size_t]
    L.mi_stream_sync.restype = ctypes.c_int
    L.mi_stream_sync.argtypes = [vp]
    L.mi_flash_attn_fwd.restype = ctypes.c_int
    L.mi_flash_attn_fwd.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i32, i32]
    L.mi_flash_attn_fwd_scaled.restype = ctypes.c_int
    L.mi_flash_attn_fwd_scaled.argtypes = L.mi_flash_attn_fwd.argtypes + [ctypes.c_float]
    L.mi_flash_attn_bwd_scaled.restype = ctypes.c_int
    L.mi_flash_attn_bwd.restype = ctypes.c_int
    L.mi_flash_attn_bwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64,
                                    i64, i32, i32, vp, ctypes.c_size_t]
    L.mi_flash_attn_bwd_scaled.argtypes = L.mi_flash_attn_bwd.argtypes + [ctypes.c_float]
    L.mi_flash_attn_bwd_workspace_size.restype = ctypes.c_size_t
    L.mi_flash_attn_bwd_workspace_size.argtypes = [i64, i64, i64]
    L.mi_cross_entropy.restype = ctypes.c_int
    L.mi_cross_entropy.argtypes = [vp, vp, i32, i64, vp, i64, i64, ctypes.c_float, vp, vp, vp,
                                   i32, i64]
    L.mi_lm_head_xent_workspace_size.restype = ctypes.c_size_t
    L.mi_lm_head_xent_workspace_size.argtypes = [i64, i64, i64, i64, i32]
    L.mi_lm_head_xent.restype = ctypes.c_int
    L.mi_lm_head_xent.argtypes = [vp, vp, i64, vp, i32, i64, vp, i64, i64, i64, ctypes.c_float, vp, vp,
                                  vp, i32, i64, vp, i32, i64, ctypes.c_float, i64, vp, ctypes.c_size_t]
    L.mi_rmsnorm_fwd.restype = ctypes.c_int
    L.mi_rmsnorm_fwd.argtypes = [vp, vp, vp, vp, i32, vp, vp, i64, i64, i64, i32, ctypes.c_float]
    L.mi_rmsnorm_bwd_workspace_size.restype = ctypes.c_size_t
    L.mi_rmsnorm_bwd_workspace_size.argtypes = [i64, i64]
    L.mi_rmsnorm_bwd.restype = ctypes.c_int
    L.mi_rmsnorm_bwd.argtypes = [vp, vp, vp, vp, i32, vp, vp, vp, i32, ctypes.c_float, i64, i64, i64,
                                 i32, ctypes.c_float, vp, ctypes.c_size_t]
    L.mi_rmsnorm_fold_weight.restype = ctypes.c_int
    L.mi_rmsnorm_fold_weight.argtypes = [vp, vp, i32, vp, i64, i64, i64, i32, vp, i64]
    L.mi_convert_matrix.restype = ctypes.c_int
    L.mi_convert_matrix.argtypes = [vp, vp, i32, i64, i64, i64, i64, i32, vp, i32, i64]
    L.mi_convert_matrices.restype = ctypes.c_int
    L.mi_convert_matrices.argtypes = [vp, ctypes.POINTER(MiConvertJob), i64]
    L.mi_profiler_enable.restype = ctypes.c_int
    L.mi_profiler_enable.argtypes = [ctypes.c_int]
    L.mi_profiler_begin_step.restype = ctypes.c_int
    L.mi_profiler_count.restype = i64
    L.mi_profiler_record.restype = ctypes.c_int
    L.mi_profiler_record.argtypes = [i64, ctypes.POINTER(MiGemmRecord)]
    L.mi_profiler_totals.restype = ctypes.c_int
    L.mi_profiler_totals.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(i64)]
    L.mi_profiler_reset.restype = ctypes.c_int
    _lib = L
    return L


def _check(fn: str, st: int):
    if st != 0:
        raise MiError(fn, st, load_library().mi_last_error().decode())


def version() -> str:
    return load_library().mi_version().decode()


def init():
    _check("mi_init", load_library().mi_init())


# ---- torch plumbing -----------------------------------------------------------

def _torch():
    import torch
    return torch


def _dt(t) -> int:
    torch = _torch()
    if t.dtype == torch.bfloat16:
        return MI_BF16
    if t.dtype == torch.float32:
        return MI_F32
    raise ValueError(f"unsupported dtype {t.dtype}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(_torch().cuda.current_stream().cuda_stream)


_scope_depth = 0


def begin_scope():
    """MetalBridge.hpp:29: calls enqueue without waiting until end_scope()."""
    global _scope_depth
    _scope_depth += 1


def end_scope():
    """MetalBridge.hpp:30: wait once for everything enqueued in the scope."""
    global _scope_depth
    _scope_depth = max(0, _scope_depth - 1)
    _check("mi_stream_sync", load_library().mi_stream_sync(_stream()))


def _finish(fn, st):
    _check(fn, st)
    if _scope_depth == 0:
        _check("mi_stream_sync", load_library().mi_stream_sync(_stream()))


# ---- general entry points -----------------------------------------------------

def _epilogue(bias=None, residual=None, ldr=None, B2=None, A2=None, row_scale=None):
    if bias is None and residual is None and B2 is None and A2 is None and row_scale is None:
        return None
    e = MiEpilogue()
    if row_scale is not None:
        e.row_scale = row_scale.data_ptr()
    if bias is not None:
        e.bias, e.bias_dtype = bias.data_ptr(), _dt(bias)
    if residual is not None:
        e.residual, e.residual_dtype = residual.data_ptr(), _dt(residual)
        e.ldr = ldr if ldr is not None else residual.shape[-1]
    if B2 is not None:
        e.B2 = B2.data_ptr()
    if A2 is not None:
        e.A2 = A2.data_ptr()
    return ctypes.byref(e)


def gemm(A, B, C, M, N, K, *, transA=False, transB=False, alpha=1.0, beta=0.0, lda=None,
         ldb=None, ldc=None, bias=None, residual=None, ldr=None, B2=None, A2=None,
         row_scale=None, workspace=None, sync=None):
    """mi_gemm on torch device tensors; C = epilogue(alpha*op(A)op(B)); row_scale: optional
    fp32 [M] tensor multiplying row m of alpha*op(A)op(B) before bias / beta / residual."""
    L = load_library()
    lda = lda if lda is not None else (M if transA else K)
    ldb = ldb if ldb is not None else (K if transB else N)
    ldc = ldc if ldc is not None else N
    ws = _ptr(workspace)
    wsb = 0 if workspace is None else workspace.numel() * workspace.element_size()
    st = L.mi_gemm(_stream(), int(transA), int(transB), M, N, K, alpha, _ptr(A), lda, _ptr(B),
                   ldb, _dt(A), beta, _ptr(C), ldc, _dt(C),
                   _epilogue(bias, residual, ldr, B2, A2, row_scale), ws, wsb)
    if sync is None:
        _finish("mi_gemm", st)
    else:
        _check("mi_gemm", st)


def make_batch(batch, heads=1, a=(0, 0, 1), b=(0, 0, 1), c=(0, 0, 1), r=(0, 0), k_segments=1,
               seg_a=0, seg_b=0, causal=MI_CAUSAL_NONE, mask_value=0.0) -> MiBatch:
    d = MiBatch()
    d.batch, d.heads = batch, heads
    d.a_outer, d.a_inner, d.a_group = a
    d.b_outer, d.b_inner, d.b_group = b
    d.c_outer, d.c_inner, d.c_group = c
    d.r_outer, d.r_inner = r
    d.k_segments, d.seg_a, d.seg_b = k_segments, seg_a, seg_b
    d.causal, d.mask_value = causal, mask_value
    return d


def gemm_batched(A, B, C, M, N, K, batch: MiBatch, *, transA=False, transB=False, alpha=1.0,
                 beta=0.0, lda=None, ldb=None, ldc=None, bias=None, residual=None, ldr=None,
                 B2=None, A2=None, workspace=None, sync=None):
    """mi_gemm_batched on torch device tensors (GQA head map, K segments, causal)."""
    L = load_library()
    lda = lda if lda is not None else (M if transA else K)
    ldb = ldb if ldb is not None else (K if transB else N)
    ldc = ldc if ldc is not None else N
    ws = _ptr(workspace)
    wsb = 0 if workspace is None else workspace.numel() * workspace.element_size()
    st = L.mi_gemm_batched(_stream(), int(transA), int(transB), M, N, K, alpha, _ptr(A), lda,
                           _ptr(B), ldb, _dt(A), beta, _ptr(C), ldc, _dt(C), ctypes.byref(batch),
                           _epilogue(bias, residual, ldr, B2, A2), ws, wsb)
    if sync is None:
        _finish("mi_gemm_batched", st)
    else:
        _check("mi_gemm_batched", st)


def describe(transA, transB, M, N, K, dtype_in=MI_BF16, batch=1, epi_mode=0, workspace_bytes=0):
    """Text description of the kernel the planner picks for this problem."""
    buf = ctypes.create_string_buffer(160)
    _check("mi_gemm_describe", load_library().mi_gemm_describe(
        int(transA), int(transB), M, N, K, dtype_in, batch, epi_mode, workspace_bytes, buf, 160))
    return buf.value.decode()


def workspace_size(transA, transB, M, N, K, dtype_in=MI_BF16, dtype_c=MI_F32, batch=1) -> int:
    return int(load_library().mi_gemm_workspace_size(int(transA), int(transB), M, N, K, dtype_in,
                                                     dtype_c, batch))


_WS_POOL = {}


def _pooled_workspace(transA, transB, M, N, K, A, C):
    """Split-K workspace for the reference-named calls: one fp32 buffer per device,
    grown to the largest size a call has asked for (the C++ bridge keeps the same pool)."""
    need = workspace_size(transA, transB, M, N, K, _dt(A), _dt(C))
    if need == 0:
        return None
    ws = _WS_POOL.get(C.device)
    if ws is None or ws.numel() * 4 < need:
        ws = _torch().empty((need + 3) // 4, dtype=_torch().float32, device=C.device)
        _WS_POOL[C.device] = ws
    return ws


# ---- reference-named entry points (MetalBridge.hpp) ---------------------------

def gemm_bf16(A, B, C, M, N, K, transA=False, transB=False, is_forward=False):
    """MetalBridge.hpp:39-42. bf16 in/out: C[M,N] = op(A) op(B). No-op if a size is 0."""
    if M == 0 or N == 0 or K == 0:
        return
    gemm(A, B, C, M, N, K, transA=transA, transB=transB,
         workspace=_pooled_workspace(transA, transB, M, N, K, A, C))


def fused_swiglu_gemm(gate_proj, up_proj, B, C, M, N, K):
    """MetalBridge.hpp:44-46: C = (SiLU(gate) * up) @ B (fused_swiglu_gemm.metal:48-77).
    With the pooled workspace holding SiLU(gate) * up, mi_gemm writes it in one pass and
    runs the plain GEMM on it (as the C++ bridge does)."""
    if M == 0 or N == 0 or K == 0:
        return
    ws = None
    if gate_proj.dtype == _torch().bfloat16:
        need = (M * K * 2 + 255) // 256 * 256 + workspace_size(0, 0, M, N, K, MI_BF16, _dt(C))
        ws = _WS_POOL.get(C.device)
        if ws is None or ws.numel() * 4 < need:
            ws = _torch().empty((need + 3) // 4, dtype=_torch().float32, device=C.device)
            _WS_POOL[C.device] = ws
    gemm(gate_proj, B, C, M, N, K, A2=up_proj, workspace=ws)


def gemm_ffn(a, b_gate, b_up, c, M, N, K):
    """MetalBridge.hpp:119-120: C = SiLU(A Bg) * (A Bu) (gemm_ffn.metal:160-181)."""
    if M == 0 or N == 0 or K == 0:
        return
    gemm(a, b_gate, c, M, N, K, B2=b_up)


def gemm_proj(a, b, c, M, N, K):
    """MetalBridge.hpp:121 (cblas_sgemm NN, MetalBridge.mm:695-697), on the GPU."""
    if M == 0 or N == 0 or K == 0:
        return
    gemm(a, b, c, M, N, K, workspace=_pooled_workspace(0, 0, M, N, K, a, c))


def gemm_backward(a_transposed, b, c, M, N, K, accumulate=False):
    """MetalBridge.hpp:122-123: C[M,N] = A^T B, A stored [K,M] (overwrites, MetalBridge.mm:1928).

    accumulate=True gives the engine's dW semantics C += A^T B (Transformer.cpp:236,
    gemm_backward.metal:104-115); C may then be fp32.
    """
    if M == 0 or N == 0 or K == 0:
        return
    gemm(a_transposed, b, c, M, N, K, transA=True, beta=1.0 if accumulate else 0.0,
         workspace=_pooled_workspace(1, 0, M, N, K, a_transposed, c))


def gemm_proj_trans_b(a, b_transposed, c, M, N, K):
    """MetalBridge.hpp:124-125: C = A B^T, B stored [N,K]."""
    if M == 0 or N == 0 or K == 0:
        return
    gemm(a, b_transposed, c, M, N, K, transB=True,
         workspace=_pooled_workspace(0, 1, M, N, K, a, c))


def residual_add(a, b, n=None):
    """MetalBridge.hpp:78: a[i] += b[i] (residual_add.metal:27)."""
    n = a.numel() if n is None else n
    _finish("mi_residual_add", load_library().mi_residual_add(_stream(), _ptr(a), _ptr(b), n,
                                                              _dt(a)))


# ---- GEMM profiler (gemm_profiler.hpp:18-117, MetalBridge.hpp:141-145) ----------

class GemmProfiler:
    """Per-call GEMM records with GPU times (HIP events around each call's kernels,
    kept by the library); same methods as the reference's GemmProfiler singleton.
    Recording is off until enable()."""

    _inst = None

    @classmethod
    def instance(cls):
        if cls._inst is None:
            cls._inst = cls()
        return cls._inst

    def enable(self, on=True):
        return bool(load_library().mi_profiler_enable(1 if on else 0))

    def begin_step(self):
        _check("mi_profiler_begin_step", load_library().mi_profiler_begin_step())

    def records(self):
        """[{M, N, K, transA, transB, batch, splits, elapsed_ms, kernel}] in call order."""
        L = load_library()
        out = []
        for i in range(L.mi_profiler_count()):
            r = MiGemmRecord()
            _check("mi_profiler_record", L.mi_profiler_record(i, ctypes.byref(r)))
            out.append(dict(M=r.M, N=r.N, K=r.K, transA=bool(r.transA), transB=bool(r.transB),
                            batch=r.batch, splits=r.splits, elapsed_ms=r.gpu_ms,
                            kernel=r.kernel.decode()))
        return out

    @staticmethod
    def op_name(M, N, K, tA, tB):
        return {(False, False): "forward (NN)", (False, True): "input gradient (NT)",
                (True, False): "weight gradient (TN)"}.get((bool(tA), bool(tB)), "TT")

    def summary(self):
        """Records aggregated per (M, N, K, tA, tB), largest GPU time first."""
        agg = {}
        for r in self.records():
            key = (r["M"], r["N"], r["K"], r["transA"], r["transB"])
            a = agg.setdefault(key, dict(M=r["M"], N=r["N"], K=r["K"], transA=r["transA"],
                                         transB=r["transB"], kernel=r["kernel"], calls=0, ms=0.0,
                                         flop=0.0))
            a["calls"] += 1
            a["ms"] += r["elapsed_ms"]
            a["flop"] += 2.0 * r["M"] * r["N"] * r["K"] * r["batch"]
        rows = sorted(agg.values(), key=lambda a: -a["ms"])
        for a in rows:
            a["op"] = self.op_name(a["M"], a["N"], a["K"], a["transA"], a["transB"])
            a["tflops"] = a["flop"] / (a["ms"] * 1e-3) / 1e12 if a["ms"] > 0 else 0.0
        return rows

    def print_summary(self, step_gpu_ms):
        rows = self.summary()
        total = sum(a["ms"] for a in rows)
        print(f"GEMM PROFILER  (step GPU time {step_gpu_ms:.3f} ms, GEMM GPU time {total:.3f} ms)")
        print(f"{'operation':22s} {'M':>6s} {'N':>6s} {'K':>6s} {'calls':>5s} {'GPU ms':>10s} "
              f"{'TFLOP/s':>9s}  kernel")
        for a in rows:
            print(f"{a['op']:22s} {a['M']:6d} {a['N']:6d} {a['K']:6d} {a['calls']:5d} "
                  f"{a['ms']:10.4f} {a['tflops']:9.1f}  {a['kernel']}")


def _totals():
    ms, n = ctypes.c_double(), ctypes.c_int64()
    _check("mi_profiler_totals", load_library().mi_profiler_totals(ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value


def accum_gpu_time_ms():
    """MetalBridge.hpp:141: GPU time of the recorded GEMM calls since the last reset."""
    return _totals()[0]


def count_gpu_calls():
    """MetalBridge.hpp:143: number of recorded GEMM calls since the last reset."""
    return _totals()[1]


def reset_profile_stats():
    """MetalBridge.hpp:145."""
    _check("mi_profiler_reset", load_library().mi_profiler_reset())


# ---- Tensor::matmul mirror ------------------------------------------------------

def matmul_shape(a_shape, b_shape):
    """Tensor.cpp:174-209 shape rules; ValueError carries the reference's messages."""
    ra, rb = len(a_shape), len(b_shape)
    if ra < 2 or rb < 2:
        raise ValueError("Matmul requires at least 2 dimensions")
    if rb == 2 and ra != 2:
        if a_shape[-1] != b_shape[0]:
            raise ValueError("Inner dimensions must match for projection")
        return tuple(a_shape[:-1]) + (b_shape[1],)
    if ra != rb:
        raise ValueError("Batch size must match for matrix multiplication")
    for i in range(ra - 2):
        if a_shape[i] != b_shape[i]:
            raise ValueError("Batch dimension must match for matmul")
    if a_shape[-1] != b_shape[-2]:
        raise ValueError("Inner dimensions must match for matmul")
    return tuple(a_shape[:-1]) + (b_shape[-1],)


def matmul(a, b):
    """Tensor::matmul: result dtype = a's dtype, zero-initialised then written."""
    torch = _torch()
    shape = matmul_shape(tuple(a.shape), tuple(b.shape))
    if a.dtype != b.dtype:
        raise ValueError("Matmul operands must share a dtype")
    a = a.contiguous()
    b = b.contiguous()
    out = torch.zeros(shape, dtype=a.dtype, device=a.device)
    if b.dim() == 2 and a.dim() != 2:
        K, N = b.shape
        M = a.numel() // K if K else math.prod(a.shape[:-1])
        gemm(a, b, out, M, N, K, workspace=_pooled_workspace(0, 0, M, N, K, a, out))
    else:
        M, K, N = a.shape[-2], a.shape[-1], b.shape[-1]
        nb = math.prod(a.shape[:-2])
        bt = make_batch(nb, 1, a=(M * K, 0, 1), b=(K * N, 0, 1), c=(M * N, 0, 1))
        gemm_batched(a, b, out, M, N, K, bt)
    return out


# ---- GQA attention composed from the batched GEMM forms ------------------------

def softmax_causal_(S, T):
    """In-place causal row softmax of S [..., T, T] (Attention.cpp:261-266)."""
    rows = S.numel() // T
    _check("mi_softmax_causal", load_library().mi_softmax_causal(_stream(), _ptr(S), rows, T, T,
                                                                 _dt(S)))


def softmax_bwd_(P, dP, T, scale):
    """dP <- P * (dP - rowsum(P * dP)) * scale (Attention.cpp:336-345)."""
    rows = P.numel() // T
    _check("mi_softmax_bwd", load_library().mi_softmax_bwd(_stream(), _ptr(P), _ptr(dP), rows, T,
                                                           T, scale, _dt(P)))


def attention_forward(Q4, K4, V4, out_dtype=None):
    """Q4 [B,nH,T,d], K4/V4 [B,nKV,T,d] -> (O [B,T,nH*d], P [B,nH,T,T]).

    S = Q K^T / sqrt(d) (NT, kv map, causal output mask), softmax, O = P V (NN,
    kv map, causal K skipping) written straight into the [B,T,nH*d] layout.
    """
    torch = _torch()
    Bn, nH, T, d = Q4.shape
    nKV = K4.shape[1]
    g = nH // nKV
    dt = Q4.dtype
    S = torch.empty((Bn, nH, T, T), dtype=dt, device=Q4.device)
    bt = make_batch(Bn * nH, nH, a=(nH * T * d, T * d, 1), b=(nKV * T * d, T * d, g),
                    c=(nH * T * T, T * T, 1), causal=MI_CAUSAL_OUT_LOWER, mask_value=-math.inf)
    gemm_batched(Q4, K4, S, T, T, d, bt, transB=True, alpha=1.0 / math.sqrt(d), sync=False)
    softmax_causal_(S, T)
    O = torch.empty((Bn, T, nH * d), dtype=out_dtype or dt, device=Q4.device)
    bt = make_batch(Bn * nH, nH, a=(nH * T * T, T * T, 1), b=(nKV * T * d, T * d, g),
                    c=(T * nH * d, d, 1), causal=MI_CAUSAL_A_LOWER)
    gemm_batched(S, V4, O, T, d, T, bt, ldc=nH * d, sync=False)
    _finish("attention_forward", 0)
    return O, S


def flash_kernel_dim(d):
    """Head dimension of the fused kernels that run head_dim d: 64 (the reference kernels'
    compiled size, flash_attn_fwd.metal:31) and 128 natively; another multiple of 8 below
    128 on operands padded with zero columns to the next of them; 0 otherwise."""
    if d <= 0 or d % 8 or d > 128:
        return 0
    return 64 if d <= 64 else 128


def flash_attn_fwd(Q4, K4, V4, O=None, lse=None, causal=True, layout="bthd", sync=None):
    """Fused forward (metal_bridge::flash_attn_fwd, MetalBridge.hpp:49-51; Attention.cpp:236-280):
    Q4 [B,nH,T,d], K4/V4 [B,nKV,T,d] bf16 -> O [B,T,nH*d] (layout "bthd", the CPU path's)
    or [B,nH,T,d] ("bhtd", the Metal kernel's).  lse: optional fp32 [B,nH,T] tensor that
    receives each row's log-sum-exp of the scaled scores. Returns O."""
    torch = _torch()
    Bn, nH, T, d = Q4.shape
    nKV = K4.shape[1]
    for t in (Q4, K4, V4):
        if t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise ValueError("Q, K, V must be contiguous bf16 tensors")
    kd = flash_kernel_dim(d)
    if kd and kd != d:
        # the next larger kernel on rows padded with zero columns, at the scale of d
        pad = lambda t: torch.nn.functional.pad(t, (0, kd - d)).contiguous()
        Qp, Kp, Vp = pad(Q4), pad(K4), pad(V4)  # held until the kernel has been queued
        Op = torch.empty((Bn, nH, T, kd), dtype=torch.bfloat16, device=Q4.device)
        st = load_library().mi_flash_attn_fwd_scaled(
            _stream(), _ptr(Qp), _ptr(Kp), _ptr(Vp), _ptr(Op), _ptr(lse), Bn, nH, nKV, T,
            kd, int(bool(causal)), MI_ATTN_O_BHTD, 1.0 / math.sqrt(d))
        _check("mi_flash_attn_fwd_scaled", st)
        res = Op[..., :d]
        res = res.permute(0, 2, 1, 3).reshape(Bn, T, nH * d) if layout == "bthd" else res
        if O is None:
            O = res.contiguous()
        else:
            O.copy_(res.reshape(O.shape))
        if sync is None and _scope_depth == 0:
            torch.cuda.synchronize(Q4.device)
        return O
    if O is None:
        shape = (Bn, T, nH * d) if layout == "bthd" else (Bn, nH, T, d)
        O = torch.empty(shape, dtype=torch.bfloat16, device=Q4.device)
    code = MI_ATTN_O_BTHD if layout == "bthd" else MI_ATTN_O_BHTD
    st = load_library().mi_flash_attn_fwd(_stream(), _ptr(Q4), _ptr(K4), _ptr(V4), _ptr(O),
                                          _ptr(lse), Bn, nH, nKV, T, d, int(bool(causal)), code)
    if sync is None:
        _finish("mi_flash_attn_fwd", st)
    else:
        _check("mi_flash_attn_fwd", st)
    return O


def flash_attn_bwd(Q4, K4, V4, O, dO, lse, causal=True, layout="bthd", sync=None, workspace="auto"):
    """Fused backward (metal_bridge::fused_attn_bwd, MetalBridge.hpp:54-57; Attention.cpp:292-348)
    from the forward's O and lse: returns (dQ [B,nH,T,d], dK, dV [B,nKV,T,d]), bf16, dK/dV
    summed over the query heads of each KV head. O and dO in `layout` ("bthd" or "bhtd").
    workspace: "auto" allocates the dS^T workspace (dQ as one batched GEMM), None runs the
    dQ kernel instead, or a device tensor of at least mi_flash_attn_bwd_workspace_size bytes."""
    torch = _torch()
    Bn, nH, T, d = Q4.shape
    nKV = K4.shape[1]
    for t in (Q4, K4, V4, O, dO):
        if t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise ValueError("Q, K, V, O, dO must be contiguous bf16 tensors")
    kd = flash_kernel_dim(d)
    if kd and kd != d:
        # the next larger kernels on rows padded with zero columns, at the scale of d
        pad = lambda t: torch.nn.functional.pad(t, (0, kd - d)).contiguous()
        if layout == "bthd":
            padl = lambda t: pad(t.reshape(Bn, T, nH, d)).reshape(Bn, T, nH * kd)
        else:
            padl = pad
        dQp = torch.empty((Bn, nH, T, kd), dtype=torch.bfloat16, device=Q4.device)
        dKp = torch.empty((Bn, nKV, T, kd), dtype=torch.bfloat16, device=Q4.device)
        dVp = torch.empty_like(dKp)
        delta = torch.empty((Bn, nH, T), dtype=torch.float32, device=Q4.device)
        code = MI_ATTN_O_BTHD if layout == "bthd" else MI_ATTN_O_BHTD
        if isinstance(workspace, str) and workspace == "auto":
            nbytes = load_library().mi_flash_attn_bwd_workspace_size(Bn, nH, T)
            workspace = torch.empty((nbytes // 2,), dtype=torch.bfloat16, device=Q4.device) if nbytes else None
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        Qp, Kp, Vp, Op, dOp = pad(Q4), pad(K4), pad(V4), padl(O), padl(dO)  # held until queued
        st = load_library().mi_flash_attn_bwd_scaled(
            _stream(), _ptr(Qp), _ptr(Kp), _ptr(Vp), _ptr(Op), _ptr(dOp), _ptr(lse),
            _ptr(dQp), _ptr(dKp), _ptr(dVp), _ptr(delta), Bn, nH, nKV, T, kd, int(bool(causal)), code,
            _ptr(workspace), ws_bytes, 1.0 / math.sqrt(d))
        _check("mi_flash_attn_bwd_scaled", st)
        out = (dQp[..., :d].contiguous(), dKp[..., :d].contiguous(), dVp[..., :d].contiguous())
        if sync is None and _scope_depth == 0:
            torch.cuda.synchronize(Q4.device)
        return out
    dQ = torch.empty_like(Q4)
    dK = torch.empty_like(K4)
    dV = torch.empty_like(V4)
    delta = torch.empty((Bn, nH, T), dtype=torch.float32, device=Q4.device)
    code = MI_ATTN_O_BTHD if layout == "bthd" else MI_ATTN_O_BHTD
    if isinstance(workspace, str) and workspace == "auto":
        nbytes = load_library().mi_flash_attn_bwd_workspace_size(Bn, nH, T)
        workspace = torch.empty((nbytes // 2,), dtype=torch.bfloat16, device=Q4.device) if nbytes else None
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    st = load_library().mi_flash_attn_bwd(_stream(), _ptr(Q4), _ptr(K4), _ptr(V4), _ptr(O),
                                          _ptr(dO), _ptr(lse), _ptr(dQ), _ptr(dK), _ptr(dV),
                                          _ptr(delta), Bn, nH, nKV, T, d, int(bool(causal)), code,
                                          _ptr(workspace), ws_bytes)
    if sync is None:
        _finish("mi_flash_attn_bwd", st)
    else:
        _check("mi_flash_attn_bwd", st)
    return dQ, dK, dV


def attention_backward(Q4, K4, V4, dO, P, grad_dtype=None):
    """Batched backward products (Attention.cpp:292-348) -> (dQ4, dK4, dV4).

    dV = P^T dO and dK = dS^T Q run as one product per (b, kv head) whose K loop
    covers the nH/nKV query heads of the group (the KV-group reduction).
    """
    torch = _torch()
    Bn, nH, T, d = Q4.shape
    nKV = K4.shape[1]
    g = nH // nKV
    dt = Q4.dtype
    gd = grad_dtype or dt
    scale = 1.0 / math.sqrt(d)
    # dV[b,kv] = sum_{h in group} P[b,h]^T dO[b,:,h]   (TN, K = g segments of T)
    dV = torch.empty(V4.shape, dtype=gd, device=Q4.device)
    bt = make_batch(Bn * nKV, nKV, a=(nH * T * T, g * T * T, 1), b=(T * nH * d, g * d, 1),
                    c=(nKV * T * d, T * d, 1), k_segments=g, seg_a=T * T, seg_b=d,
                    causal=MI_CAUSAL_A_UPPER)
    gemm_batched(P, dO, dV, T, d, T, bt, transA=True, ldb=nH * d, sync=False)
    # dP[b,h] = dO[b,:,h] V[b,kv]^T   (NT, kv map)
    dP = torch.empty((Bn, nH, T, T), dtype=dt, device=Q4.device)
    bt = make_batch(Bn * nH, nH, a=(T * nH * d, d, 1), b=(nKV * T * d, T * d, g),
                    c=(nH * T * T, T * T, 1), causal=MI_CAUSAL_OUT_LOWER, mask_value=0.0)
    gemm_batched(dO, V4, dP, T, T, d, bt, transB=True, lda=nH * d, sync=False)
    # dS = P * (dP - rowsum(P * dP)) * scale, in place over dP
    softmax_bwd_(P, dP, T, scale)
    # dQ[b,h] = dS[b,h] K[b,kv]   (NN, kv map, causal K skipping)
    dQ = torch.empty(Q4.shape, dtype=gd, device=Q4.device)
    bt = make_batch(Bn * nH, nH, a=(nH * T * T, T * T, 1), b=(nKV * T * d, T * d, g),
                    c=(nH * T * d, T * d, 1), causal=MI_CAUSAL_A_LOWER)
    gemm_batched(dP, K4, dQ, T, d, T, bt, sync=False)
    # dK[b,kv] = sum_{h in group} dS[b,h]^T Q[b,h]   (TN, K = g segments of T)
    dK = torch.empty(K4.shape, dtype=gd, device=Q4.device)
    bt = make_batch(Bn * nKV, nKV, a=(nH * T * T, g * T * T, 1), b=(nH * T * d, g * T * d, 1),
                    c=(nKV * T * d, T * d, 1), k_segments=g, seg_a=T * T, seg_b=T * d,
                    causal=MI_CAUSAL_A_UPPER)
    gemm_batched(dP, Q4, dK, T, d, T, bt, transA=True, sync=False)
    _finish("attention_backward", 0)
    return dQ, dK, dV


# ---- loss ---------------------------------------------------------------------

def cross_entropy(logits, targets, grad="new", grad_dtype=None, scale=None, sync=None,
                  row_loss=None, loss=None):
    """Softmax cross-entropy over the rows of logits [..., V] (metal_bridge::cross_entropy,
    MetalBridge.hpp:89-91; CrossEntropyLoss, Loss.cpp:43-195).

    logits: bf16 or fp32, last dimension contiguous. targets: integer tensor of the
    leading shape (a value outside [0, V) gives a NaN row loss). Returns (loss, row_loss,
    grad): loss a 1-element fp32 device tensor = scale * sum(row_loss), row_loss fp32
    [rows] = -log(max(p_target, 1e-15)), grad = scale * (softmax - onehot) shaped like
    logits. grad: "new" allocates it in grad_dtype (default fp32, the reference's),
    "inplace" overwrites the logits, None skips it, or a tensor to write into.
    scale defaults to 1 / rows, the reference's mean. row_loss ([rows] fp32) and loss ([1]
    fp32) may be given to reuse device buffers."""
    torch = _torch()
    V = logits.shape[-1]
    rows = logits.numel() // V if V else 0
    if logits.stride(-1) != 1:
        raise ValueError("logits must have a contiguous last dimension")
    L2 = logits.reshape(rows, V)
    ld = L2.stride(0) if rows > 1 else V
    tg = targets.reshape(-1).to(torch.int32).contiguous()
    if tg.numel() != rows:
        raise ValueError(f"targets has {tg.numel()} entries for {rows} rows")
    if scale is None:
        scale = 1.0 / rows if rows else 0.0
    if row_loss is None:
        row_loss = torch.empty((rows,), dtype=torch.float32, device=logits.device)
    if loss is None:
        loss = torch.empty((1,), dtype=torch.float32, device=logits.device)
    if row_loss.numel() < rows or row_loss.dtype != torch.float32 or loss.dtype != torch.float32:
        raise ValueError("row_loss must hold rows fp32 values and loss one fp32 value")
    if isinstance(grad, str) and grad == "new":
        g = torch.empty(logits.shape, dtype=grad_dtype or torch.float32, device=logits.device)
    elif isinstance(grad, str) and grad == "inplace":
        g = logits
    elif grad is None:
        g = None
    else:
        g = grad
    if g is not None:
        if g.stride(-1) != 1 or g.shape != logits.shape:
            raise ValueError("grad must match the logits' shape with a contiguous last dimension")
        ldg = g.reshape(rows, V).stride(0) if rows > 1 else V
    else:
        ldg = 0
    st = load_library().mi_cross_entropy(
        _stream(), _ptr(L2), _dt(logits), ld, _ptr(tg), rows, V, float(scale), _ptr(row_loss),
        _ptr(loss), _ptr(g), _dt(g) if g is not None else MI_F32, ldg)
    if sync is None:
        _finish("mi_cross_entropy", st)
    else:
        _check("mi_cross_entropy", st)
    return loss, row_loss, g


def lm_head_xent_workspace_size(rows, hidden, vocab, chunk=8192, dx_dtype=None) -> int:
    """Bytes of workspace lm_head_xent needs (mi_lm_head_xent_workspace_size)."""
    torch = _torch()
    dt = MI_F32 if dx_dtype == torch.float32 else MI_BF16
    return int(load_library().mi_lm_head_xent_workspace_size(rows, hidden, vocab, chunk, dt))


def lm_head_xent(X, W, targets, w_layout=0, chunk=8192, scale=None, dX="new", dx_dtype=None,
                 dW=None, dw_beta=0.0, row_loss=None, loss=None, workspace=None, sync=None):
    """LM head + cross-entropy over vocabulary chunks, no [rows, vocab] logits
    (mi_lm_head_xent; the reference's final_h.matmul(output_projection_), Transformer.cpp:
    193-194, CrossEntropyLoss, Loss.cpp:43-195, and the output projection backward,
    Transformer.cpp:600-616).

    X [rows, hidden] bf16; W bf16, [hidden, vocab] for w_layout 0 (logits = X W, the
    reference's output_projection_) or [vocab, hidden] for w_layout 1 (logits = X W^T).
    Returns (loss, row_loss, dX): dX = G W^T or G W with G = scale * (softmax - onehot);
    dX "new" allocates it in dx_dtype (default bf16), None skips it, or a tensor to write
    into. dW, if given (W's shape, bf16 or fp32), becomes dw_beta * dW + X^T G (or G^T X).
    scale defaults to 1 / rows. workspace: a device tensor of at least
    lm_head_xent_workspace_size bytes (allocated when None)."""
    torch = _torch()
    rows, hidden = X.shape
    vocab = W.shape[1] if w_layout == 0 else W.shape[0]
    if (W.shape[0] if w_layout == 0 else W.shape[1]) != hidden:
        raise ValueError(f"W {tuple(W.shape)} does not match hidden={hidden} for w_layout {w_layout}")
    for name, t in (("X", X), ("W", W)):
        if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
            raise ValueError(f"{name} must be bf16 with a contiguous last dimension")
    tg = targets.reshape(-1).to(torch.int32).contiguous()
    if tg.numel() != rows:
        raise ValueError(f"targets has {tg.numel()} entries for {rows} rows")
    if scale is None:
        scale = 1.0 / rows if rows else 0.0
    dev = X.device
    if row_loss is None:
        row_loss = torch.empty((rows,), dtype=torch.float32, device=dev)
    if loss is None:
        loss = torch.empty((1,), dtype=torch.float32, device=dev)
    if isinstance(dX, str) and dX == "new":
        dX = torch.empty((rows, hidden), dtype=dx_dtype or torch.bfloat16, device=dev)
    if dX is not None and (dX.shape != X.shape or dX.stride(-1) != 1):
        raise ValueError("dX must match X's shape with a contiguous last dimension")
    if dW is not None and (dW.shape != W.shape or dW.stride(-1) != 1):
        raise ValueError("dW must match W's shape with a contiguous last dimension")
    dxt = _dt(dX) if dX is not None else MI_BF16
    need = int(load_library().mi_lm_head_xent_workspace_size(rows, hidden, vocab, chunk, dxt))
    if workspace is None:
        workspace = torch.empty((max(need, 1),), dtype=torch.uint8, device=dev)
    wsb = workspace.numel() * workspace.element_size()
    ld = lambda t: t.stride(0) if t.shape[0] > 1 else t.shape[1]  # noqa: E731
    st = load_library().mi_lm_head_xent(
        _stream(), _ptr(X), ld(X), _ptr(W), int(w_layout), ld(W), _ptr(tg), rows, hidden, vocab,
        float(scale), _ptr(row_loss), _ptr(loss), _ptr(dX), dxt, ld(dX) if dX is not None else 0,
        _ptr(dW), _dt(dW) if dW is not None else MI_F32, ld(dW) if dW is not None else 0,
        float(dw_beta), int(chunk), _ptr(workspace), wsb)
    if sync is None:
        _finish("mi_lm_head_xent", st)
    else:
        _check("mi_lm_head_xent", st)
    return loss, row_loss, dX


class CrossEntropyLoss:
    """Mirror of the reference's CrossEntropyLoss (Loss.hpp; Loss.cpp:43-195, GPU branch):
    forward(logits [B,S,V], targets [B,S]) returns the mean loss as a Python float and
    keeps the logits gradient; backward(targets) returns it ([B,S,V] fp32, scaled by
    1 / (B*S))."""

    def __init__(self):
        self._grad = None

    def forward(self, logits, targets) -> float:
        loss, _, self._grad = cross_entropy(logits, targets)
        return float(loss.item())

    def backward(self, targets=None):
        if self._grad is None:
            raise RuntimeError("CrossEntropyLoss.backward before forward")
        return self._grad


# ---- RMSNorm ------------------------------------------------------------------

def _rows_of(t, what):
    """(rows, dims, ld) of a row-major [..., dims] tensor whose rows share one stride."""
    dims = t.shape[-1]
    if t.stride(-1) != 1:
        raise ValueError(f"{what} must have a contiguous last dimension")
    if t.dim() == 2:
        return t.shape[0], dims, (t.stride(0) if t.shape[0] > 1 else dims)
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous (or 2-D with a row stride)")
    return t.numel() // dims if dims else 0, dims, dims


def rms_norm_forward(x, weight, eps=1e-5, residual=None, out=None, rstd=None, sync=None):
    """RMSNorm forward (metal_bridge::rms_norm_forward, MetalBridge.hpp:60-61; RMSNorm.cpp:48-75):
    y = x / sqrt(mean(x^2) + eps) * weight over the last dimension. With residual, first
    x += residual in place (metal_bridge::fused_add_norm, Transformer.cpp:150-158). x, residual,
    out: bf16 or fp32 with one row stride; weight [dims] bf16 or fp32; rstd: optional fp32 [rows]
    tensor receiving 1/rms. out may be x; out=False computes only the residual add and rstd
    (the norm folded into the next GEMM: rms_norm_matmul). Returns y (or rstd)."""
    torch = _torch()
    rows, dims, ld = _rows_of(x, "x")
    if out is False:
        if rstd is None:
            raise ValueError("the statistic-only form needs rstd")
        if residual is not None and (residual.dtype != x.dtype or _rows_of(residual, "residual") != (rows, dims, ld)):
            raise ValueError("residual must match x's dtype, shape and row stride")
        st = load_library().mi_rmsnorm_fwd(_stream(), _ptr(x), _ptr(residual), _ptr(weight), _dt(weight),
                                           None, _ptr(rstd), rows, dims, ld, _dt(x), float(eps))
        (_finish if sync is None else _check)("mi_rmsnorm_fwd", st)
        return rstd
    if out is None:
        out = torch.empty_strided(x.shape, x.stride(), dtype=x.dtype, device=x.device)
    for t, n in ((out, "out"), (residual, "residual")):
        if t is not None and (t.dtype != x.dtype or _rows_of(t, n) != (rows, dims, ld)):
            raise ValueError(f"{n} must match x's dtype, shape and row stride")
    st = load_library().mi_rmsnorm_fwd(_stream(), _ptr(x), _ptr(residual), _ptr(weight), _dt(weight),
                                       _ptr(out), _ptr(rstd), rows, dims, ld, _dt(x), float(eps))
    if sync is None:
        _finish("mi_rmsnorm_fwd", st)
    else:
        _check("mi_rmsnorm_fwd", st)
    return out


def rms_norm_fold_weight(weight, W, out=None, sync=None):
    """W'[k, n] = weight[k] * W[k, n] (mi_rmsnorm_fold_weight): the RMSNorm weight moved into
    the rows of the GEMM's B operand (engine layout W[in, out]). out may be W. Returns W'."""
    torch = _torch()
    if W.dim() != 2 or W.stride(1) != 1 or weight.numel() != W.shape[0]:
        raise ValueError("W must be a row-major [K, N] matrix and weight [K]")
    if out is None:
        out = torch.empty_like(W)
    st = load_library().mi_rmsnorm_fold_weight(_stream(), _ptr(weight), _dt(weight), _ptr(W), W.stride(0),
                                               W.shape[0], W.shape[1], _dt(W), _ptr(out), out.stride(0))
    (_finish if sync is None else _check)("mi_rmsnorm_fold_weight", st)
    return out


def rms_norm_matmul(x, norm_weight, W, C=None, eps=1e-5, residual=None, folded=None, rstd=None,
                    workspace=None, sync=None):
    """rmsnorm(x [+= residual]) @ W with the norm folded into the GEMM (Transformer.cpp:147-162,
    Attention.cpp:196-201: fused_add_norm / rms_norm_forward, then the QKV or gate/up matmul):
    one row statistic (rstd = 1/rms, x += residual in place first) and one GEMM on x itself,
    C = diag(rstd) x W' with W' = diag(norm_weight) W and rstd as the GEMM's row scale; the
    normalised activations are never written. folded: W' from rms_norm_fold_weight (computed
    here when not given). x [M, K] bf16 or fp32, W [K, N]. Returns C [M, N] in x's dtype."""
    torch = _torch()
    M, K = x.shape
    N = W.shape[1]
    if rstd is None:
        rstd = torch.empty((M,), dtype=torch.float32, device=x.device)
    rms_norm_forward(x, norm_weight, eps=eps, residual=residual, out=False, rstd=rstd, sync=False)
    if folded is None:
        folded = rms_norm_fold_weight(norm_weight, W, sync=False)
    if C is None:
        C = torch.empty((M, N), dtype=x.dtype, device=x.device)
    gemm(x, folded, C, M, N, K, lda=x.stride(0), ldb=folded.stride(0), row_scale=rstd,
         workspace=workspace, sync=sync)
    return C


def rms_norm_backward(dy, x, weight, eps=1e-5, residual_grad=None, dx=None, dw=None, dw_beta=0.0,
                      want_dw=True, sync=None):
    """RMSNorm backward (metal_bridge::rms_norm_backward, MetalBridge.hpp:62-64; RMSNorm.cpp:77-180):
    dx = (dy*w - xhat*mean(dy*w*xhat)) / rms [+ residual_grad] (metal_bridge::fused_backward_add_norm,
    Transformer.cpp:441-466), dw = dw_beta*dw + sum over rows of dy*xhat. dw (fp32 [dims] unless
    given) is allocated when want_dw; dx may be dy. Returns (dx, dw or None)."""
    torch = _torch()
    rows, dims, ld = _rows_of(x, "x")
    if dx is None:
        dx = torch.empty_strided(x.shape, x.stride(), dtype=x.dtype, device=x.device)
    for t, n in ((dy, "dy"), (dx, "dx"), (residual_grad, "residual_grad")):
        if t is not None and (t.dtype != x.dtype or _rows_of(t, n) != (rows, dims, ld)):
            raise ValueError(f"{n} must match x's dtype, shape and row stride")
    ws = None
    if want_dw or dw is not None:
        if dw is None:
            dw = torch.zeros((dims,), dtype=torch.float32, device=x.device)
        nbytes = load_library().mi_rmsnorm_bwd_workspace_size(rows, dims)
        ws = torch.empty((max(nbytes, 4) // 4,), dtype=torch.float32, device=x.device)
    st = load_library().mi_rmsnorm_bwd(
        _stream(), _ptr(dy), _ptr(x), _ptr(weight), _dt(weight), _ptr(residual_grad), _ptr(dx),
        _ptr(dw), _dt(dw) if dw is not None else MI_F32, float(dw_beta), rows, dims, ld, _dt(x),
        float(eps), _ptr(ws), 0 if ws is None else ws.numel() * 4)
    if sync is None:
        _finish("mi_rmsnorm_bwd", st)
    else:
        _check("mi_rmsnorm_bwd", st)
    return dx, dw


class RMSNorm:
    """Mirror of the reference's RMSNorm (RMSNorm.hpp; RMSNorm.cpp:31-180): weight [dims]
    (bf16, initialised to 1 as RMSNorm.cpp:31), forward(x) -> y, backward(grad_output, input,
    grad_weight) -> grad_input with grad_weight (fp32 [dims]) accumulated, as the CPU path does."""

    def __init__(self, dims, eps=1e-5, device="cuda", dtype=None):
        torch = _torch()
        self.eps = float(eps)
        self.weight = torch.ones((dims,), dtype=dtype or torch.bfloat16, device=device)

    def forward(self, x):
        if x.dim() < 2:
            raise ValueError("Input tensor must have at least 2 dimensions")
        if x.shape[-1] != self.weight.shape[0]:
            raise ValueError("Input tensor last dimension must match RMSNorm dims")
        return rms_norm_forward(x, self.weight, self.eps)

    def backward(self, grad_output, input, grad_weight):
        if tuple(grad_output.shape) != tuple(input.shape):
            raise ValueError("grad_output and input shapes must match in RMSNorm::backward")
        if tuple(grad_weight.shape) != tuple(self.weight.shape):
            raise ValueError("grad_weight must match RMSNorm weight dimensions")
        dx, _ = rms_norm_backward(grad_output, input, self.weight, self.eps, dw=grad_weight,
                                  dw_beta=1.0)
        return dx


# ---- checkpoint weights ---------------------------------------------------------

_ST_DTYPES = {"F32": (MI_F32, 4), "BF16": (MI_BF16, 2), "F16": (MI_F16, 2)}


def read_safetensors_header(path):
    """(header dict, payload offset) of a safetensors file (Checkpoint.cpp:390-400): 8-byte
    little-endian length (at most 10 MiB, as the reference), then the JSON header."""
    import json
    import struct

    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: shorter than 8 bytes")
        (n,) = struct.unpack("<Q", raw)
        if n == 0 or n > (10 << 20):
            raise ValueError(f"{path}: bad header length {n}")
        head = json.loads(f.read(n).decode("utf-8"))
    return head, 8 + n


def convert_matrix(src, src_dtype, src_ld, row0, rows, cols, transpose, dst, sync=None):
    """mi_convert_matrix: rows [row0, row0+rows) x [0, cols) of a device source matrix
    (raw bytes of dtype MI_F32 / MI_BF16 / MI_F16, leading dimension src_ld) into dst
    (fp32 or bf16 tensor), transposed or not (Checkpoint.cpp:77-83, 407-530)."""
    ld_dst = rows if transpose else cols
    st = load_library().mi_convert_matrix(_stream(), _ptr(src), src_dtype, src_ld, row0, rows, cols,
                                          int(bool(transpose)), _ptr(dst), _dt(dst), ld_dst)
    if sync is None:
        _finish("mi_convert_matrix", st)
    else:
        _check("mi_convert_matrix", st)
    return dst


def convert_jobs(jobs):
    """A ctypes array of mi_convert_job from (src, src_dtype, src_ld, row0, rows, cols,
    transpose, dst) tuples (src and dst device tensors; the destination dtype and leading
    dimension come from dst); built once, it can be handed to convert_matrices any number
    of times."""
    arr = (MiConvertJob * len(jobs))()
    for a, (src, sdt, sld, row0, rows, cols, tr, dst) in zip(arr, jobs):
        a.src, a.src_dtype, a.transpose = src.data_ptr(), sdt, int(bool(tr))
        a.src_ld, a.row0, a.rows, a.cols = sld, row0, rows, cols
        a.dst, a.dst_dtype, a.reserved = dst.data_ptr(), _dt(dst), 0
        a.dst_ld = dst.stride(0) if dst.dim() == 2 else (rows if tr else cols)
    return arr


def convert_matrices(jobs, sync=None):
    """mi_convert_matrices: several mi_convert_matrix conversions in as few launches as
    their dtype pairs allow (Checkpoint.cpp:532-570).  jobs: a list of tuples as for
    convert_jobs, or an array it returned."""
    arr = jobs if isinstance(jobs, ctypes.Array) else convert_jobs(jobs)
    st = load_library().mi_convert_matrices(_stream(), arr, len(arr))
    if sync is None:
        _finish("mi_convert_matrices", st)
    else:
        _check("mi_convert_matrices", st)


def engine_weight_shapes(cfg):
    """Engine names and [in, out] shapes of a model's weights (Checkpoint.cpp:147-174).
    cfg: dict with n_layers, hidden_dim, n_heads, n_kv_heads, head_dim, intermediate_dim,
    vocab_size."""
    H, V, I = cfg["hidden_dim"], cfg["vocab_size"], cfg["intermediate_dim"]
    q, kv = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    shapes = {"token_embeddings": (V, H), "output_projection": (H, V), "final_norm.weight": (H,)}
    for l in range(cfg["n_layers"]):
        p = f"layers.{l}."
        shapes.update({p + "attn_norm.weight": (H,), p + "attn.Wq": (H, q), p + "attn.Wk": (H, kv),
                       p + "attn.Wv": (H, kv), p + "attn.Wo": (q, H), p + "ffn_norm.weight": (H,),
                       p + "w_gate": (H, I), p + "w_up": (H, I), p + "w_down": (I, H)})
    return shapes


def weight_sources(cfg, python_format):
    """For every engine tensor: (file tensor, file shape, row0, rows, transpose). The
    Python/MLX layout is nn.Linear [out, in] with fused attention.wqkv and feed_forward.w12
    (Checkpoint.cpp:532-570); the engine layout is the engine's own (:147-174)."""
    H, V, I = cfg["hidden_dim"], cfg["vocab_size"], cfg["intermediate_dim"]
    q, kv = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    src = {}
    if python_format:
        src["token_embeddings"] = ("tok_embeddings.weight", (V, H), 0, V, False)
        src["output_projection"] = ("output.weight", (V, H), 0, V, True)
        src["final_norm.weight"] = ("norm.weight", (H,), 0, 1, False)
        for l in range(cfg["n_layers"]):
            p = f"layers.{l}."
            src[p + "attn_norm.weight"] = (p + "attention_norm.weight", (H,), 0, 1, False)
            src[p + "ffn_norm.weight"] = (p + "ffn_norm.weight", (H,), 0, 1, False)
            src[p + "attn.Wo"] = (p + "attention.wo.weight", (H, q), 0, H, True)
            src[p + "w_down"] = (p + "feed_forward.w3.weight", (H, I), 0, H, True)
            fq = (q + 2 * kv, H)
            src[p + "attn.Wq"] = (p + "attention.wqkv.weight", fq, 0, q, True)
            src[p + "attn.Wk"] = (p + "attention.wqkv.weight", fq, q, kv, True)
            src[p + "attn.Wv"] = (p + "attention.wqkv.weight", fq, q + kv, kv, True)
            src[p + "w_gate"] = (p + "feed_forward.w12.weight", (2 * I, H), 0, I, True)
            src[p + "w_up"] = (p + "feed_forward.w12.weight", (2 * I, H), I, I, True)
    else:
        for name, shape in engine_weight_shapes(cfg).items():
            src[name] = (name, shape, 0, shape[0] if len(shape) == 2 else 1, False)
    return src


def load_weights(path, cfg, dtype=None, device="cuda"):
    """Mirror of the model part of Checkpoint::load (Checkpoint.cpp:331-388, 532-570): reads a
    Python/MLX or an engine safetensors file into new device tensors in the engine layout
    (dict keyed by the engine names), dtype bf16 (default) or fp32. Each file tensor's bytes
    go to the device once; slicing, transposing and widening run in mi_convert_matrices, one
    call per file tensor (the row ranges of a fused wqkv or w12 together)."""
    import numpy as np
    torch = _torch()

    dtype = dtype or torch.bfloat16
    head, payload = read_safetensors_header(path)
    python_format = "tok_embeddings.weight" in head
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    staged = {}
    pending = []
    out = {}
    for name, shape in engine_weight_shapes(cfg).items():
        fname, fshape, row0, rows, transpose = weight_sources(cfg, python_format)[name]
        ent = head.get(fname)
        if ent is None:
            raise KeyError(f"tensor '{fname}' not found in {path}")
        if tuple(ent["shape"]) != tuple(fshape):
            raise ValueError(f"tensor '{fname}' has shape {ent['shape']}, expected {list(fshape)}")
        if ent["dtype"] not in _ST_DTYPES:
            raise ValueError(f"tensor '{fname}' has dtype {ent['dtype']}")
        code, es = _ST_DTYPES[ent["dtype"]]
        b, e = ent["data_offsets"]
        if e - b != int(np.prod(fshape)) * es or payload + e > mm.size:
            raise ValueError(f"tensor '{fname}' has a byte range that does not match its shape")
        if fname not in staged:
            if pending:
                convert_matrices(pending, sync=False)
                pending = []
            staged = {fname: torch.from_numpy(np.array(mm[payload + b: payload + e])).to(device)}
        cols = fshape[-1]
        dst = torch.empty(shape, dtype=dtype, device=device)
        pending.append((staged[fname], code, cols, row0, rows, cols, transpose,
                        dst if dst.dim() == 2 else dst.view(1, -1)))
        out[name] = dst
    if pending:
        convert_matrices(pending, sync=False)
    _finish("load_weights", 0)
    return out
