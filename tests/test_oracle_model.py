"""Pins of the model-level CPU oracle (oracle/model_oracle.cpp) without a GPU.

  - rmsnorm: a constant row maps to sign(c)·w (closed form), and rows match float64 numpy;
  - silu_mul: silu(0) = 0, silu(x) -> x and -> 0 at the extremes, float64 numpy elsewhere;
  - forward: a model with no layers gives logits = output·rmsnorm(embedding row) (numpy); layers
    whose wo and w_down are zero leave the residual stream unchanged; and a two-layer model
    matches an independent float64 numpy forward (numpy matmul on the dequantized weights,
    rotation of adjacent pairs, causal softmax over the f16-rounded cache) within f32 rounding —
    a wrong step order, a missing residual add, rope on the wrong tensor or a cache row off by
    one each give O(1) errors.
"""
from __future__ import annotations

import numpy as np
import pytest

import gguf_blocks as gb
import llama_synth as ls

CFG = dict(n_layer=2, n_embd=256, n_head=2, n_head_kv=1, head_dim=128, n_ff=512, n_vocab=300,
           rope_theta=10000.0, rms_eps=1e-5)


def test_rmsnorm(oracle_mod):
    rng = np.random.default_rng(0)
    w = rng.standard_normal(64).astype(np.float32)
    x = np.full((1, 64), -3.0, np.float32)
    np.testing.assert_allclose(oracle_mod.rmsnorm(x, w, 1e-5)[0], -w, rtol=1e-5)
    x = rng.standard_normal((5, 64)).astype(np.float32)
    want = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-5) * w
    np.testing.assert_allclose(oracle_mod.rmsnorm(x, w, 1e-5), want, rtol=2e-6, atol=1e-6)


def test_silu_mul(oracle_mod):
    g = np.array([0.0, 40.0, -40.0, 1.0, -2.5], np.float32)
    u = np.array([3.0, 2.0, 2.0, 1.0, 1.0], np.float32)
    got = oracle_mod.silu_mul(g, u)
    assert got[0] == 0.0 and abs(got[1] - 80.0) < 1e-4 and abs(got[2]) < 1e-15
    gd = g.astype(np.float64)
    np.testing.assert_allclose(got[3:], (gd / (1 + np.exp(-gd)) * u)[3:], rtol=1e-6)


def _dequant(orc, t):
    typ, raw = t
    be, bb = gb.BLOCK[gb.type_id(typ)]
    n_in = raw.shape[1] // bb * be
    return orc.dequant_rows(typ, raw, n_in).astype(np.float64)


def _np_forward(orc, m, tokens):
    """Independent float64 forward over the dequantized weights (cache rounded to f16)."""
    c = m["cfg"]
    hd, H, HKV = c["head_dim"], c["n_head"], c["n_head_kv"]
    inv = m["rope_inv_freq"]
    E = _dequant(orc, m["tok_embd"])
    O = _dequant(orc, m["output"])
    Ls = [{k: (_dequant(orc, v) if isinstance(v, tuple) else v.astype(np.float64)) for k, v in L.items()}
          for L in m["layers"]]

    def norm(x, w):
        return x / np.sqrt((x * x).mean() + c["rms_eps"]) * w

    def rope(x, nh, pos):
        x = x.reshape(nh, hd // 2, 2).copy()
        ang = (np.float32(pos) * inv).astype(np.float64)
        cth, sth = np.cos(ang), np.sin(ang)
        a, b = x[..., 0].copy(), x[..., 1].copy()
        x[..., 0], x[..., 1] = a * cth - b * sth, a * sth + b * cth
        return x.reshape(-1)

    K = [[] for _ in Ls]
    V = [[] for _ in Ls]
    out = []
    for pos, tok in enumerate(tokens):
        x = E[tok].copy()
        for l, L in enumerate(Ls):
            h = norm(x, L["attn_norm"])
            q, k, v = rope(L["wq"] @ h, H, pos), rope(L["wk"] @ h, HKV, pos), L["wv"] @ h
            K[l].append(k.astype(np.float16).astype(np.float64))
            V[l].append(v.astype(np.float16).astype(np.float64))
            Kl, Vl = np.array(K[l]), np.array(V[l])
            att = np.zeros(H * hd)
            for hh in range(H):
                kv = hh // (H // HKV)
                s = Kl[:, kv * hd:(kv + 1) * hd] @ q[hh * hd:(hh + 1) * hd] / np.sqrt(hd)
                p = np.exp(s - s.max())
                att[hh * hd:(hh + 1) * hd] = (p / p.sum()) @ Vl[:, kv * hd:(kv + 1) * hd]
            x = x + L["wo"] @ att
            h = norm(x, L["ffn_norm"])
            g, u = L["w_gate"] @ h, L["w_up"] @ h
            x = x + L["w_down"] @ (g / (1 + np.exp(-g)) * u)
        out.append(O @ norm(x, m["output_norm"]))
    return out


def test_forward_no_layers(oracle_mod):
    cfg = dict(CFG, n_layer=0)
    m = ls.make_model(cfg, "Q8_0", seed=1, tied=False)
    o = oracle_mod.ForwardOracle(m, n_ctx=4)
    got = o.forward(7, 0)
    E, O = _dequant(oracle_mod, m["tok_embd"]), _dequant(oracle_mod, m["output"])
    x = E[7]
    want = O @ (x / np.sqrt((x * x).mean() + cfg["rms_eps"]) * m["output_norm"])
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 * np.abs(want).max())


def test_forward_zero_residual_branches(oracle_mod):
    m = ls.make_model(CFG, "F16", seed=2, tied=False)
    for L in m["layers"]:
        L["wo"] = ("F16", np.zeros_like(L["wo"][1]))
        L["w_down"] = ("F16", np.zeros_like(L["w_down"][1]))
    m0 = dict(m, cfg=dict(CFG, n_layer=0), layers=[])
    a = oracle_mod.ForwardOracle(m, n_ctx=4).forward(5, 0)
    b = oracle_mod.ForwardOracle(m0, n_ctx=4).forward(5, 0)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("types", ["F16", "Q4_0"])
def test_forward_matches_float64_numpy(oracle_mod, types):
    m = ls.make_model(CFG, types, seed=3, tied=True)
    tokens = [3, 17, 299, 0, 42]
    o = oracle_mod.ForwardOracle(m, n_ctx=8)
    got = [o.forward(t, p) for p, t in enumerate(tokens)]
    want = _np_forward(oracle_mod, m, tokens)
    for g, w in zip(got, want):
        rel = np.linalg.norm(g - w) / np.linalg.norm(w)
        assert rel < 2e-5, rel
