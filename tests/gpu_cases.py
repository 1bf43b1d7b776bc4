"""Helpers shared by the GPU parity tests: seeded inputs, operand layouts, checks."""
import numpy as np

TOL_F32 = 1e-4   # north-star tolerance for fp32 inputs (max relative error)
TOL_BF16 = 1e-2  # bf16 inputs vs the float64 oracle fed the same bf16-rounded inputs


def inputs(oracle, shape, seed, std=1.0, bf16=True):
    """N(0, std) from the repo generator, rounded to bf16 (RNE) when bf16 is set."""
    x = oracle.normal(shape, seed, 0.0, std)
    return oracle.round_bf16(x) if bf16 else x


def layout(op, trans):
    """Memory layout of the logical operand op [R, C] for a transpose flag."""
    return np.ascontiguousarray(op.T) if trans else np.ascontiguousarray(op)


def to_dev(x, dev, bf16):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(dev, torch.bfloat16 if bf16 else torch.float32)


def host(t):
    return t.float().cpu().numpy().astype(np.float64)


def check(got, ref, tol, what=""):
    from oracle import max_rel_err

    err = max_rel_err(got, ref)
    assert np.isfinite(err) and err <= tol, f"{what}: max rel err {err:.3e} > {tol:.0e}"
    return err


def checksums(a_op, b_op):
    """Column and row checksums of C = a_op @ b_op, float64, O(MK + KN):
    1^T C = (1^T A) B   and   C 1 = A (B 1)."""
    a = a_op.astype(np.float64)
    b = b_op.astype(np.float64)
    return a.sum(axis=0) @ b, a @ b.sum(axis=1)


def sample_rows(M, n=8, seed=0):
    rng = np.random.default_rng(seed)
    rows = set(rng.choice(M, size=min(n, M), replace=False).tolist())
    rows |= {0, M - 1}
    return np.array(sorted(rows), dtype=np.int64)


def dense_attention(q, k, v, causal):
    """float64 softmax(Q K^T / sqrt(d)) V and the row log-sum-exp, [B,nH,T,d] layouts
    (the closed form; the causal case is also checked against the oracle)."""
    Bn, nH, T, d = q.shape
    g = nH // k.shape[1]
    kk = np.repeat(k.astype(np.float64), g, axis=1)
    vv = np.repeat(v.astype(np.float64), g, axis=1)
    s = np.einsum("bhqc,bhkc->bhqk", q.astype(np.float64), kk) / np.sqrt(d)
    if causal:
        s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
    mx = s.max(axis=-1, keepdims=True)
    e = np.exp(s - mx)
    lse = (np.log(e.sum(axis=-1)) + mx[..., 0])
    o = np.einsum("bhqk,bhkc->bhqc", e / e.sum(axis=-1, keepdims=True), vv)
    return o, lse


def dense_attention_bwd(q, k, v, do, causal):
    """float64 closed form of the backward: dV = P^T dO, dS = P (dO V^T - rowsum(dO O)),
    dQ = dS K / sqrt(d), dK = dS^T Q / sqrt(d), dK and dV summed over a KV head's query
    heads.  do is [B, T, nH*d]."""
    Bn, nH, T, d = q.shape
    nKV = k.shape[1]
    g = nH // nKV
    qq = q.astype(np.float64)
    kk = np.repeat(k.astype(np.float64), g, axis=1)
    vv = np.repeat(v.astype(np.float64), g, axis=1)
    s = np.matmul(qq, kk.transpose(0, 1, 3, 2)) / np.sqrt(d)
    if causal:
        s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    o = np.matmul(p, vv)
    g4 = do.astype(np.float64).reshape(Bn, T, nH, d).transpose(0, 2, 1, 3)
    ds = p * (np.matmul(g4, vv.transpose(0, 1, 3, 2)) - (g4 * o).sum(axis=-1, keepdims=True))
    dq = np.matmul(ds, kk) / np.sqrt(d)
    dk = (np.matmul(ds.transpose(0, 1, 3, 2), qq) / np.sqrt(d)).reshape(Bn, nKV, g, T, d).sum(2)
    dv = np.matmul(p.transpose(0, 1, 3, 2), g4).reshape(Bn, nKV, g, T, d).sum(2)
    return dq, dk, dv
