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


def random_blocks(t, n_out: int, n_in: int, scale: float, rng) -> np.ndarray:
    """Valid random GGUF rows, generated directly as bytes (fast, for full-size bench models):
    block scales near `scale` (values of magnitude ~scale), random quants. F16/F32 fall back to
    quantize() of normal values."""
    tid = gb.type_id(t)
    be, bb = gb.BLOCK[tid]
    if be == 1:
        return gb.quantize(t, (rng.standard_normal((n_out, n_in)) * scale).astype(np.float32))
    nb = n_in // be
    out = rng.integers(0, 256, size=(n_out, nb, bb), dtype=np.uint8)
    d = (scale * (0.5 + rng.random((n_out, nb)))).astype(np.float32)
    if tid == 2:    # Q4_0: d * (nibble - 8), |values| <= 8d
        d /= 8
    elif tid == 3:  # Q4_1: d * nibble + m
        d /= 8
        out[..., 2:4] = (-8 * d).astype(np.float16).view(np.uint8).reshape(n_out, nb, 2)
    elif tid == 8:  # Q8_0: d * int8
        d /= 128
    elif tid == 14:  # Q6_K: d * scale_j * (q - 32), scales int8 in [1, 127]
        sc = rng.integers(1, 128, size=(n_out, nb, 16), dtype=np.int8)
        out[..., 192:208] = sc.view(np.uint8)
        d /= 32 * 64
    off = 208 if tid == 14 else 0
    out[..., off:off + 2] = d.astype(np.float16).view(np.uint8).reshape(n_out, nb, 2)
    return out.reshape(n_out, nb * bb)


def make_bench_model(cfg: dict, t: str = "Q4_0", seed: int = 0) -> dict:
    """A full-size model with random-byte weights of type t (tied embeddings, as Llama-3.2-3B)."""
    rng = np.random.default_rng(seed)
    ne, hd, nf, nv = cfg["n_embd"], cfg["head_dim"], cfg["n_ff"], cfg["n_vocab"]
    qd, kvd = cfg["n_head"] * hd, cfg["n_head_kv"] * hd

    def w(n_out, n_in, scale):
        return (t, random_blocks(t, n_out, n_in, scale, rng))

    m = {"cfg": dict(cfg), "rope_inv_freq": rope_inv_freq(cfg["rope_theta"], hd), "layers": []}
    m["tok_embd"] = w(nv, ne, 1.0)
    m["output"] = m["tok_embd"]
    m["output_norm"] = np.ones(ne, np.float32)
    for _ in range(cfg["n_layer"]):
        m["layers"].append({
            "attn_norm": np.ones(ne, np.float32), "ffn_norm": np.ones(ne, np.float32),
            "wq": w(qd, ne, 1 / np.sqrt(ne)), "wk": w(kvd, ne, 1 / np.sqrt(ne)), "wv": w(kvd, ne, 1 / np.sqrt(ne)),
            "wo": w(ne, qd, 0.5 / np.sqrt(qd)), "w_gate": w(nf, ne, 1 / np.sqrt(ne)),
            "w_up": w(nf, ne, 1 / np.sqrt(ne)), "w_down": w(ne, nf, 0.5 / np.sqrt(nf)),
        })
    return m


def weight_bytes(m: dict) -> int:
    """Bytes of all weight tensors (the embedding table counted once when tied)."""
    total = m["tok_embd"][1].nbytes + (0 if m["output"] is m["tok_embd"] else m["output"][1].nbytes)
    for L in m["layers"]:
        total += sum(v[1].nbytes for k, v in L.items() if isinstance(v, tuple))
    return total
