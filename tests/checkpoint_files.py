"""Synthetic safetensors checkpoints for the loader tests: a Python/MLX-layout file
(nn.Linear [out, in], fused attention.wqkv and feed_forward.w12, Checkpoint.cpp:532-570)
and an engine-layout file (Checkpoint.cpp:147-174), written with the safetensors library."""
import numpy as np

CFG = dict(n_layers=2, hidden_dim=64, n_heads=4, n_kv_heads=2, head_dim=16, intermediate_dim=96,
           vocab_size=200)


def _t(torch, shape, seed, dtype):
    g = np.random.default_rng(seed)
    return torch.from_numpy(g.normal(0, 1, shape).astype(np.float32)).to(dtype)


def write_python_file(path, cfg=CFG, dtypes=None):
    """MLX names; dtypes cycles over the given torch dtypes (default bf16, f16, f32)."""
    import torch
    from safetensors.torch import save_file

    dts = dtypes or [torch.bfloat16, torch.float16, torch.float32]
    H, V, I = cfg["hidden_dim"], cfg["vocab_size"], cfg["intermediate_dim"]
    q, kv = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    shapes = {"tok_embeddings.weight": (V, H), "output.weight": (V, H), "norm.weight": (H,)}
    for l in range(cfg["n_layers"]):
        p = f"layers.{l}."
        shapes.update({p + "attention_norm.weight": (H,), p + "ffn_norm.weight": (H,),
                       p + "attention.wo.weight": (H, q), p + "feed_forward.w3.weight": (H, I),
                       p + "attention.wqkv.weight": (q + 2 * kv, H),
                       p + "feed_forward.w12.weight": (2 * I, H)})
    tensors = {n: _t(torch, s, 1000 + i, dts[i % len(dts)]) for i, (n, s) in enumerate(shapes.items())}
    save_file(tensors, path, metadata={"format": "mlx"})
    return tensors


def write_engine_file(path, cfg=CFG, dtype=None):
    import torch
    from safetensors.torch import save_file

    H, V, I = cfg["hidden_dim"], cfg["vocab_size"], cfg["intermediate_dim"]
    q, kv = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    shapes = {"token_embeddings": (V, H), "output_projection": (H, V), "final_norm.weight": (H,)}
    for l in range(cfg["n_layers"]):
        p = f"layers.{l}."
        shapes.update({p + "attn_norm.weight": (H,), p + "attn.Wq": (H, q), p + "attn.Wk": (H, kv),
                       p + "attn.Wv": (H, kv), p + "attn.Wo": (q, H), p + "ffn_norm.weight": (H,),
                       p + "w_gate": (H, I), p + "w_up": (H, I), p + "w_down": (I, H)})
    tensors = {n: _t(torch, s, 2000 + i, dtype or torch.float32) for i, (n, s) in enumerate(shapes.items())}
    save_file(tensors, path, metadata={"format": "pt"})
    return tensors


def expected_engine(tensors, cfg=CFG):
    """The engine-layout float32 arrays a Python/MLX file should load as, computed with
    torch slicing and transposes from the tensors the safetensors library wrote."""
    H, I = cfg["hidden_dim"], cfg["intermediate_dim"]
    q, kv = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    f = {k: v.float() for k, v in tensors.items()}
    out = {"token_embeddings": f["tok_embeddings.weight"], "output_projection": f["output.weight"].t(),
           "final_norm.weight": f["norm.weight"]}
    for l in range(cfg["n_layers"]):
        p = f"layers.{l}."
        wqkv, w12 = f[p + "attention.wqkv.weight"], f[p + "feed_forward.w12.weight"]
        out.update({p + "attn_norm.weight": f[p + "attention_norm.weight"],
                    p + "ffn_norm.weight": f[p + "ffn_norm.weight"],
                    p + "attn.Wo": f[p + "attention.wo.weight"].t(),
                    p + "w_down": f[p + "feed_forward.w3.weight"].t(),
                    p + "attn.Wq": wqkv[:q].t(), p + "attn.Wk": wqkv[q:q + kv].t(),
                    p + "attn.Wv": wqkv[q + kv:].t(),
                    p + "w_gate": w12[:I].t(), p + "w_up": w12[I:].t()})
    return {k: v.contiguous().numpy() for k, v in out.items()}
