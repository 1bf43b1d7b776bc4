"""numpy/ctypes front end of the CPU oracle (mi_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. Product code never imports it.

Every function here forwards to mi_oracle.c, whose header lists the reference
file:line each routine restates (Tensor.hpp:16-27, MetalBridge.mm:691-701,
gemm_bf16.metal:45,63, gemm_backward.metal:104-115, gemm_ffn.metal:160-181,
fused_swiglu_gemm.metal:48-77, Activations.cpp:31-75, residual_add.metal:27,
Attention.cpp:236-348, Loss.cpp:43-195, RMSNorm.cpp:40-180), except
checkpoint_weights, which restates the checkpoint loader (Checkpoint.cpp) in numpy.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmi_oracle.so")
_lib = None

_i64 = ctypes.c_int64
_dbl = ctypes.c_double
_vp = ctypes.c_void_p


def build() -> str:
    """Compile libmi_oracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.mo_f32_to_bf16_trunc.restype = ctypes.c_uint16
        L.mo_f32_to_bf16_trunc.argtypes = [ctypes.c_float]
        L.mo_f32_to_bf16_rne.restype = ctypes.c_uint16
        L.mo_f32_to_bf16_rne.argtypes = [ctypes.c_float]
        L.mo_bf16_to_f32.restype = ctypes.c_float
        L.mo_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.mo_to_bf16.argtypes = [_vp, _vp, _i64, ctypes.c_int]
        L.mo_from_bf16.argtypes = [_vp, _vp, _i64]
        L.mo_round_bf16.argtypes = [_vp, _i64, ctypes.c_int]
        L.mo_fill_normal.argtypes = [_vp, _i64, ctypes.c_uint64, _dbl, _dbl]
        L.mo_gemm_ex.argtypes = [ctypes.c_int, ctypes.c_int, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _dbl, _vp, _i64, _vp, _vp, _i64, _vp, _dbl, _vp, _i64,
                                 _vp, _vp, _i64, ctypes.c_int, _vp, _i64, _vp, _i64]
        L.mo_attention_fwd.argtypes = [_i64] * 5 + [_vp] * 5
        L.mo_attention_bwd.argtypes = [_i64] * 5 + [_vp] * 7
        L.mo_cross_entropy.restype = _dbl
        L.mo_cross_entropy.argtypes = [_vp, _i64, _vp, _i64, _i64, _dbl, _vp, _vp]
        L.mo_rmsnorm_fwd.argtypes = [_vp, _vp, _vp, _i64, _i64, _dbl, ctypes.c_int, _vp, _vp]
        L.mo_rmsnorm_bwd.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _dbl, _vp, _vp]
        L.mo_sgemm_omp.argtypes = [ctypes.c_int, ctypes.c_int, _i64, _i64, _i64, ctypes.c_float,
                                   _vp, _i64, _vp, _i64, ctypes.c_float, _vp, _i64]
        L.mo_num_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(_vp)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


# ---- bf16 ------------------------------------------------------------------

def to_bf16(x, rne: bool = True) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().mo_to_bf16(_p(x), _p(out), x.size, int(rne))
    return out


def from_bf16(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().mo_from_bf16(_p(h), _p(out), h.size)
    return out


def round_bf16(x, rne: bool = True) -> np.ndarray:
    """fp32 copy of x holding bf16-representable values."""
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    lib().mo_round_bf16(_p(y), y.size, int(rne))
    return y


def normal(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    lib().mo_fill_normal(_p(out), n, seed, mean, std)
    return out.reshape(shape)


# ---- GEMM ------------------------------------------------------------------

def gemm(tA, tB, M, N, K, A, B, *, lda=None, ldb=None, alpha=1.0, beta=0.0, C0=None,
         ldc0=None, bias=None, R=None, ldr=None, mode=0, A2=None, B2=None, nseg=1,
         segA=0, segB=0, rows=None) -> np.ndarray:
    """float64 result of the epilogue GEMM (see mo_gemm_ex in mi_oracle.c).

    A, B, A2, B2, C0, bias, R are flat-indexable fp32 arrays in the layouts given
    by the transpose flags and leading dimensions. K is the per-segment length.
    rows: optional int64 list of output rows to compute (sampled oracle).
    """
    A, B, A2, B2, C0, bias, R = map(_f32, (A, B, A2, B2, C0, bias, R))
    if lda is None:
        lda = M if tA else K
    if ldb is None:
        ldb = K if tB else N
    rws = None if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    nr = M if rws is None else rws.size
    out = np.empty((nr, N), dtype=np.float64)
    lib().mo_gemm_ex(int(tA), int(tB), M, N, K, nseg, segA, segB, alpha, _p(A), lda, _p(A2),
                     _p(B), ldb, _p(B2), beta, _p(C0), ldc0 if ldc0 is not None else N,
                     _p(bias), _p(R), ldr if ldr is not None else N, mode, _p(out), N,
                     _p(rws), 0 if rws is None else rws.size)
    return out


def attention_fwd(Q4, K4, V4, want_p: bool = False):
    """Attention.cpp:236-280. Q4 [B,nH,T,d], K4/V4 [B,nKV,T,d] -> O [B,T,nH*d] (f64)."""
    Q4, K4, V4 = map(_f32, (Q4, K4, V4))
    Bn, nH, T, d = Q4.shape
    nKV = K4.shape[1]
    O = np.empty((Bn, T, nH * d), dtype=np.float64)
    P = np.empty((Bn, nH, T, T), dtype=np.float64) if want_p else None
    lib().mo_attention_fwd(Bn, nH, nKV, T, d, _p(Q4), _p(K4), _p(V4), _p(O), _p(P))
    return (O, P) if want_p else O


def attention_bwd(Q4, K4, V4, dO):
    """Attention.cpp:292-348. dO [B,T,nH*d] -> (dQ4, dK4, dV4) float64."""
    Q4, K4, V4, dO = map(_f32, (Q4, K4, V4, dO))
    Bn, nH, T, d = Q4.shape
    nKV = K4.shape[1]
    dQ = np.empty(Q4.shape, dtype=np.float64)
    dK = np.empty(K4.shape, dtype=np.float64)
    dV = np.empty(V4.shape, dtype=np.float64)
    lib().mo_attention_bwd(Bn, nH, nKV, T, d, _p(Q4), _p(K4), _p(V4), _p(dO),
                           _p(dQ), _p(dK), _p(dV))
    return dQ, dK, dV


def cross_entropy(logits, targets, scale=None, want_grad=True):
    """Loss.cpp:43-195. logits [rows, V] (fp32 values), targets [rows] integers ->
    (loss, row_loss [rows], grad [rows, V] or None), float64; scale defaults to 1/rows."""
    x = _f32(logits)
    rows, V = x.shape
    t = np.ascontiguousarray(targets, dtype=np.int64).reshape(-1)
    if scale is None:
        scale = 1.0 / rows
    row_loss = np.empty((rows,), dtype=np.float64)
    grad = np.empty((rows, V), dtype=np.float64) if want_grad else None
    loss = lib().mo_cross_entropy(_p(x), V, _p(t), rows, V, float(scale), _p(row_loss), _p(grad))
    return loss, row_loss, grad


def rmsnorm_fwd(x, w, eps=1e-5, residual=None, round_bf16=False):
    """RMSNorm.cpp:40-75 (+ the residual add of fused_add_norm). x [rows, dims] ->
    (y float64, rstd float64 [rows], x_after (x + residual as stored, float32))."""
    xs = np.array(x, dtype=np.float32, order="C", copy=True)
    rows, dims = xs.shape
    r = _f32(residual)
    y = np.empty((rows, dims), dtype=np.float64)
    rstd = np.empty((rows,), dtype=np.float64)
    lib().mo_rmsnorm_fwd(_p(xs), _p(r), _p(_f32(w)), rows, dims, float(eps), int(bool(round_bf16)),
                         _p(y), _p(rstd))
    return y, rstd, xs


def rmsnorm_bwd(dy, x, w, eps=1e-5, residual_grad=None, dw0=None):
    """RMSNorm.cpp:77-180 (+ the residual gradient of fused_backward_add_norm).
    -> (dx float64 [rows, dims], dw float64 [dims] = dw0 + sum_rows dy * xhat)."""
    dy, x = _f32(dy), _f32(x)
    rows, dims = x.shape
    dx = np.empty((rows, dims), dtype=np.float64)
    dw = np.zeros((dims,), dtype=np.float64) if dw0 is None else np.array(dw0, dtype=np.float64)
    lib().mo_rmsnorm_bwd(_p(dy), _p(x), _p(_f32(w)), _p(_f32(residual_grad)), rows, dims, float(eps),
                         _p(dx), _p(dw))
    return dx, dw


def bf16_bits_to_f32(bits):
    """Checkpoint.cpp:28-33 (bf16_to_f32): the 16 bits as the high half of an fp32."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def engine_matrix(bits, row0, rows):
    """Rows row0 .. row0+rows-1 of a bf16 [out, in] file matrix (as uint16 bits) in the
    engine's [in, out] float32 layout (Checkpoint.cpp:407-535: load_python_fused_tensor's
    row range, bf16_to_f32, transpose_matrix)."""
    return bf16_bits_to_f32(bits[row0:row0 + rows]).T.copy()


def checkpoint_weights(path, cfg):
    """Checkpoint.cpp:28-83, 390-570 in numpy: the model tensors of a safetensors file (a
    Python/MLX file holding "tok_embeddings.weight", or an engine file) as float32 arrays in
    the engine layout, keyed by the engine names. bf16 and f16 widen exactly (bf16_to_f32:
    the 16 bits as the high half of an fp32; f16_to_f32); [out, in] matrices are transposed
    (transpose_matrix) and the fused wqkv / w12 are cut into row ranges first
    (load_python_fused_tensor)."""
    import json
    import struct

    raw = np.fromfile(path, dtype=np.uint8)
    (n,) = struct.unpack("<Q", raw[:8].tobytes())
    head = json.loads(raw[8:8 + n].tobytes().decode("utf-8"))
    payload = 8 + n

    def tensor(name):
        ent = head[name]
        b, e = ent["data_offsets"]
        byts = raw[payload + b: payload + e]
        if ent["dtype"] == "BF16":
            v = bf16_bits_to_f32(byts.view(np.uint16))
        elif ent["dtype"] == "F16":
            v = byts.view(np.float16).astype(np.float32)
        else:
            v = byts.view(np.float32).copy()
        return v.reshape(ent["shape"])

    H, V, I = cfg["hidden_dim"], cfg["vocab_size"], cfg["intermediate_dim"]
    q, kv = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    out = {}
    if "tok_embeddings.weight" in head:
        out["token_embeddings"] = tensor("tok_embeddings.weight")
        out["output_projection"] = tensor("output.weight").T.copy()
        out["final_norm.weight"] = tensor("norm.weight")
        for l in range(cfg["n_layers"]):
            p = f"layers.{l}."
            out[p + "attn_norm.weight"] = tensor(p + "attention_norm.weight")
            out[p + "ffn_norm.weight"] = tensor(p + "ffn_norm.weight")
            out[p + "attn.Wo"] = tensor(p + "attention.wo.weight").T.copy()
            out[p + "w_down"] = tensor(p + "feed_forward.w3.weight").T.copy()
            wqkv = tensor(p + "attention.wqkv.weight")
            out[p + "attn.Wq"] = wqkv[:q].T.copy()
            out[p + "attn.Wk"] = wqkv[q:q + kv].T.copy()
            out[p + "attn.Wv"] = wqkv[q + kv:q + 2 * kv].T.copy()
            w12 = tensor(p + "feed_forward.w12.weight")
            out[p + "w_gate"] = w12[:I].T.copy()
            out[p + "w_up"] = w12[I:2 * I].T.copy()
    else:
        names = ["token_embeddings", "output_projection", "final_norm.weight"]
        for l in range(cfg["n_layers"]):
            p = f"layers.{l}."
            names += [p + k for k in ("attn_norm.weight", "attn.Wq", "attn.Wk", "attn.Wv", "attn.Wo",
                                      "ffn_norm.weight", "w_gate", "w_up", "w_down")]
        for k in names:
            out[k] = tensor(k)
    return out


def sgemm_omp(tA, tB, M, N, K, A, B, C=None, alpha=1.0, beta=0.0, lda=None, ldb=None):
    """fp32 OpenMP SGEMM (CPU baseline), cblas_sgemm row-major semantics."""
    A, B = _f32(A), _f32(B)
    if lda is None:
        lda = M if tA else K
    if ldb is None:
        ldb = K if tB else N
    if C is None:
        C = np.zeros((M, N), dtype=np.float32)
    lib().mo_sgemm_omp(int(tA), int(tB), M, N, K, alpha, _p(A), lda, _p(B), ldb, beta, _p(C), N)
    return C


def num_threads() -> int:
    return lib().mo_num_threads()


# ---- error metrics (tolerances are defined in the tests that use them) -------

def max_rel_err(y, ref) -> float:
    """Normwise max relative error: max|y - ref| / max|ref|."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref)) if ref.size else 0.0
    num = np.max(np.abs(y - ref)) if ref.size else 0.0
    return float(num / den) if den > 0 else float(num)


def l2_rel_err(y, ref) -> float:
    """test_gpu_kernels.cpp:36-46 L2-relative error."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = float(np.sum(ref * ref))
    return 0.0 if den == 0.0 else float(np.sqrt(np.sum((y - ref) ** 2) / den))
