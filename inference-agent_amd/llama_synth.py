"""Synthetic Llama models in the GGUF tensor layout (test and bench data only).

There are no model files on the GPU box; these have the architecture of src/model.cpp:40-110
(token_embd, per-layer attn_norm/ffn_norm and the seven projections, output_norm, output or
tied embeddings, rotary frequencies as Model::load computes them) with random weights encoded
in the requested GGUF types by gguf_blocks.quantize.
"""
from __future__ import annotations

import numpy as np

import gguf_blocks as gb

# Llama-3.2-3B: 28 layers, 3072 wide, 24 Q / 8 KV heads of 128, FFN 8192,
# vocabulary 128256, rope theta 500000, rms eps 1e-5, tied embeddings.
LLAMA32_3B = dict(n_layer=28, n_embd=3072, n_head=24, n_head_kv=8, head_dim=128, n_ff=8192,
                  n_vocab=128256, rope_theta=500000.0, rms_eps=1e-5)


def rope_inv_freq(theta: float, head_dim: int) -> np.ndarray:
    """Model::load's iterated multiply (src/model.cpp:59-68), in f32."""
    scale = np.float32(np.power(np.float32(theta), np.float32(-2.0) / np.float32(head_dim)))
    out = np.empty(head_dim // 2, dtype=np.float32)
    f = np.float32(1.0)
    for i in range(head_dim // 2):
        out[i] = f
        f = np.float32(f * scale)
    return out


def make_model(cfg: dict, types: dict | str = "Q4_0", seed: int = 0, tied: bool = True) -> dict:
    """A random model. `types` maps tensor kind ("embd", "output", "wq", ..., "w_down") to a GGUF
    type name, or is one name for all projections (the embedding/output then use it too)."""
    rng = np.random.default_rng(seed)
    kinds = ("embd", "output", "wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")
    t = {k: types for k in kinds} if isinstance(types, str) else {k: types.get(k, "F16") for k in kinds}
    ne, hd, nf, nv = cfg["n_embd"], cfg["head_dim"], cfg["n_ff"], cfg["n_vocab"]
    qd, kvd = cfg["n_head"] * hd, cfg["n_head_kv"] * hd

    def w(kind, n_out, n_in, scale):
        x = (rng.standard_normal((n_out, n_in)) * scale).astype(np.float32)
        return (t[kind], gb.quantize(t[kind], x))

    def norm(n):
        return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)

    m = {"cfg": dict(cfg), "rope_inv_freq": rope_inv_freq(cfg["rope_theta"], hd), "layers": []}
    m["tok_embd"] = w("embd", nv, ne, 1.0)
    m["output"] = m["tok_embd"] if tied else w("output", nv, ne, 1.0 / np.sqrt(ne))
    m["output_norm"] = norm(ne)
    for _ in range(cfg["n_layer"]):
        m["layers"].append({
            "attn_norm": norm(ne), "ffn_norm": norm(ne),
            "wq": w("wq", qd, ne, 1.0 / np.sqrt(ne)), "wk": w("wk", kvd, ne, 1.0 / np.sqrt(ne)),
            "wv": w("wv", kvd, ne, 1.0 / np.sqrt(ne)), "wo": w("wo", ne, qd, 0.5 / np.sqrt(qd)),
            "w_gate": w("w_gate", nf, ne, 1.0 / np.sqrt(ne)), "w_up": w("w_up", nf, ne, 1.0 / np.sqrt(ne)),
            "w_down": w("w_down", ne, nf, 0.5 / np.sqrt(nf)),
        })
    return m
