"""Pins the CPU oracle (oracle/attn_oracle.cpp) before it is trusted as the checker.

The reference holds no golden vectors or known-answer tests for attention (its tests are
end-to-end diffs against llama.cpp binaries that are absent here), so each oracle function is
pinned by checks that a plausible mistake would fail:
  - f16 conversions: exhaustively against numpy's IEEE binary16 casts;
  - softmax (src/ops.cpp:234-241): closed forms;
  - decode attention (src/cpu_backend.cpp:51-69): closed forms that pin the head mapping
    kvh = h / group, the scale 1/sqrt(hd), the sign and base of the exponent, and the V sum;
    plus an f64 numpy matrix-form computation on small shapes;
  - prefill (src/backend.h:16-20): equality with successive decode steps, and causality.
"""
from __future__ import annotations

import math

import numpy as np
import pytest


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


# ---------------------------------------------------------------- f16 conversions


def test_f16_to_f32_exhaustive(oracle_mod):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle_mod.f16_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne(oracle_mod):
    rng = _rng(7)
    # random bit patterns over the whole float range, plus every f16 value and the midpoints
    # between neighbouring f16 values (ties must round to even)
    rand = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    finite = halves[np.isfinite(halves)].astype(np.float64)
    finite = np.unique(finite)
    mids = ((finite[:-1] + finite[1:]) / 2).astype(np.float32)
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.0**-25, 2.0**-24, 3 * 2.0**-26,
                     np.inf, -np.inf], dtype=np.float32)
    x = np.concatenate([rand, finite.astype(np.float32), mids, edge])
    got = oracle_mod.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    # NaN stays NaN (payload is not part of the contract)
    g = got[nan]
    assert np.all(((g & 0x7C00) == 0x7C00) & ((g & 0x03FF) != 0))


# ---------------------------------------------------------------- softmax


def test_softmax_closed_forms(oracle_mod):
    p = oracle_mod.softmax(np.array([0.0, math.log(3.0)]))
    np.testing.assert_allclose(p, [0.25, 0.75], rtol=1e-6)
    p = oracle_mod.softmax(np.full(37, 4.5))
    np.testing.assert_allclose(p, np.full(37, 1 / 37), rtol=1e-6)
    # shift invariance and a large offset (the max subtraction keeps it finite)
    x = _rng(1).standard_normal(100).astype(np.float32)
    np.testing.assert_allclose(oracle_mod.softmax(x + 1000.0), oracle_mod.softmax(x), atol=2e-6)
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(oracle_mod.softmax(x), e / e.sum(), rtol=2e-6, atol=1e-9)
    assert oracle_mod.softmax(np.array([-np.inf, 0.0]))[0] == 0.0


# ---------------------------------------------------------------- decode closed forms

H, HKV, HD = 24, 8, 128
KV = HKV * HD


def _bits(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def test_single_key_returns_v0(oracle_mod):
    rng = _rng(2)
    q = rng.standard_normal(H * HD).astype(np.float32)
    k = _bits(rng.standard_normal((1, KV)))
    v = _bits(rng.standard_normal((1, KV)))
    out = oracle_mod.attn_decode(q, k, v, H, HKV, HD, 1).reshape(H, HD)
    vf = v.view(np.float16).astype(np.float32).reshape(HKV, HD)
    for h in range(H):
        assert np.array_equal(out[h], vf[h // 3])


def test_equal_keys_give_mean_of_v(oracle_mod):
    rng = _rng(3)
    L = 50
    q = rng.standard_normal(H * HD).astype(np.float32)
    k = np.tile(_bits(rng.standard_normal((1, KV))), (L, 1))
    v = _bits(rng.standard_normal((L, KV)))
    out = oracle_mod.attn_decode(q, k, v, H, HKV, HD, L).reshape(H, HD)
    mean = v.view(np.float16).astype(np.float64).reshape(L, HKV, HD).mean(axis=0)
    for h in range(H):
        np.testing.assert_allclose(out[h], mean[h // 3], atol=2e-6)


def test_head_mapping_is_h_div_group(oracle_mod):
    # V rows constant per KV head: every Q head must return its own group's constant. A
    # mapping of h % n_head_kv (or any other) fails this.
    rng = _rng(4)
    L = 17
    consts = np.arange(1, HKV + 1, dtype=np.float32) * 0.25
    v = _bits(np.tile(np.repeat(consts, HD), (L, 1)))
    k = _bits(rng.standard_normal((L, KV)))
    q = rng.standard_normal(H * HD).astype(np.float32)
    out = oracle_mod.attn_decode(q, k, v, H, HKV, HD, L).reshape(H, HD)
    for h in range(H):
        np.testing.assert_allclose(out[h], consts[h // (H // HKV)], rtol=1e-6)


def test_two_key_logistic_pins_scale_and_exp(oracle_mod):
    # key 0 = 0, key 1 = e_0 (unit vector); q = a*e_0 -> scores 0 and a/sqrt(128);
    # p1 = 1 / (1 + exp(-a/sqrt(128))). v0 = 0, v1 = 1 -> out = p1.
    a = 3.0
    k = np.zeros((2, KV), dtype=np.float32)
    k[1, ::HD] = 1.0
    v = np.zeros((2, KV), dtype=np.float32)
    v[1, :] = 1.0
    q = np.zeros(H * HD, dtype=np.float32)
    q[::HD] = a
    out = oracle_mod.attn_decode(q, _bits(k), _bits(v), H, HKV, HD, 2)
    p1 = 1.0 / (1.0 + math.exp(-a / math.sqrt(HD)))
    np.testing.assert_allclose(out, p1, rtol=1e-6)
    # an explicit scale argument replaces 1/sqrt(hd)
    out = oracle_mod.attn_decode(q, _bits(k), _bits(v), H, HKV, HD, 2, scale=0.5)
    np.testing.assert_allclose(out, 1.0 / (1.0 + math.exp(-a * 0.5)), rtol=1e-6)


def test_dominant_key(oracle_mod):
    rng = _rng(5)
    L = 64
    k = rng.standard_normal((L, KV)).astype(np.float32) * 0.01
    q = np.ones(H * HD, dtype=np.float32)
    k[41] = 2.0  # score 256/sqrt(128)*... dominates every other key by > 40 nats
    v = rng.standard_normal((L, KV)).astype(np.float32)
    out = oracle_mod.attn_decode(q, _bits(k), _bits(v), H, HKV, HD, L).reshape(H, HD)
    v41 = _bits(v[41]).view(np.float16).astype(np.float32).reshape(HKV, HD)
    for h in range(H):
        np.testing.assert_allclose(out[h], v41[h // 3], atol=1e-6)


def _numpy_attention_f64(q, kb, vb, n_head, n_head_kv, hd, n_keys, scale):
    kf = kb[:n_keys].view(np.float16).astype(np.float64).reshape(n_keys, n_head_kv, hd)
    vf = vb[:n_keys].view(np.float16).astype(np.float64).reshape(n_keys, n_head_kv, hd)
    qh = q.astype(np.float64).reshape(n_head, hd)
    g = n_head // n_head_kv
    kg = np.repeat(kf, g, axis=1)  # [L, n_head, hd], head h -> kv head h // g
    vg = np.repeat(vf, g, axis=1)
    s = np.einsum("hd,lhd->hl", qh, kg) * scale
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return np.einsum("hl,lhd->hd", p, vg)


@pytest.mark.parametrize("n_head,n_head_kv,L", [(24, 8, 1), (24, 8, 64), (8, 8, 33), (8, 2, 40), (16, 4, 7)])
def test_decode_matches_f64_matrix_form(oracle_mod, n_head, n_head_kv, L):
    rng = _rng(100 + L)
    q = rng.standard_normal(n_head * HD).astype(np.float32)
    kb = _bits(rng.standard_normal((L, n_head_kv * HD)))
    vb = _bits(rng.standard_normal((L, n_head_kv * HD)))
    got = oracle_mod.attn_decode(q, kb, vb, n_head, n_head_kv, HD, L)
    want = _numpy_attention_f64(q, kb, vb, n_head, n_head_kv, HD, L, 1 / math.sqrt(HD))
    np.testing.assert_allclose(got.reshape(n_head, HD), want, atol=3e-6, rtol=1e-5)


def test_threads_do_not_change_bits(oracle_mod):
    rng = _rng(6)
    L = 300
    q = rng.standard_normal(H * HD).astype(np.float32)
    kb = _bits(rng.standard_normal((L, KV)))
    vb = _bits(rng.standard_normal((L, KV)))
    a = oracle_mod.attn_decode(q, kb, vb, H, HKV, HD, L, threads=1)
    b = oracle_mod.attn_decode(q, kb, vb, H, HKV, HD, L, threads=7)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------- prefill


def test_prefill_is_successive_decode_steps(oracle_mod):
    rng = _rng(8)
    pos, n = 20, 13
    q = rng.standard_normal((n, H * HD)).astype(np.float32)
    kb = _bits(rng.standard_normal((pos + n, KV)))
    vb = _bits(rng.standard_normal((pos + n, KV)))
    out = oracle_mod.attn_prefill(q, kb, vb, H, HKV, HD, pos, n, threads=4)
    for i in range(n):
        step = oracle_mod.attn_decode(q[i], kb, vb, H, HKV, HD, pos + i + 1)
        assert np.array_equal(out[i], step)


def test_prefill_is_causal(oracle_mod):
    rng = _rng(9)
    pos, n = 5, 9
    q = rng.standard_normal((n, H * HD)).astype(np.float32)
    kb = _bits(rng.standard_normal((pos + n, KV)))
    vb = _bits(rng.standard_normal((pos + n, KV)))
    base = oracle_mod.attn_prefill(q, kb, vb, H, HKV, HD, pos, n)
    i = 3  # rows > pos+i must not matter to query i
    kb2, vb2 = kb.copy(), vb.copy()
    kb2[pos + i + 1:] = _bits(rng.standard_normal((n - i - 1, KV)) * 5)
    vb2[pos + i + 1:] = _bits(rng.standard_normal((n - i - 1, KV)) * 5)
    pert = oracle_mod.attn_prefill(q, kb2, vb2, H, HKV, HD, pos, n)
    assert np.array_equal(pert[: i + 1], base[: i + 1])
    assert not np.array_equal(pert[i + 1:], base[i + 1:])
    # first query of a chunk at position 0 sees only key 0: out = v0
    out0 = oracle_mod.attn_prefill(q[:1], kb, vb, H, HKV, HD, 0, 1)[0].reshape(H, HD)
    v0 = vb[0].view(np.float16).astype(np.float32).reshape(HKV, HD)
    for h in range(H):
        assert np.array_equal(out0[h], v0[h // 3])


def test_oracle_rejects_bad_arguments(oracle_mod):
    q = np.zeros(H * HD, dtype=np.float32)
    kb = np.zeros((4, KV), dtype=np.uint16)
    with pytest.raises(ValueError):
        oracle_mod.attn_decode(q, kb, kb, 24, 7, HD, 4)  # 24 % 7 != 0
    with pytest.raises(ValueError):
        oracle_mod.attn_decode(q, kb, kb, 24, 8, HD, 0)


# --- RoPE and the KV store (src/ops.cpp:243-255, src/model.cpp:59-68, src/cpu_backend.cpp:43-49)


def test_rope_inv_freq_closed_form(oracle_mod):
    """inv_freq[i] = theta^(-2i/d) (iterated multiply: drift ~1e-6), divided by the factors."""
    for theta, d in ((10000.0, 128), (500000.0, 128), (10000.0, 64)):
        got = oracle_mod.rope_inv_freq(theta, d).astype(np.float64)
        want = theta ** (-2.0 * np.arange(d // 2) / d)
        assert got[0] == 1.0
        np.testing.assert_allclose(got, want, rtol=2e-5)
    factors = np.linspace(1.0, 8.0, 64).astype(np.float32)
    base = oracle_mod.rope_inv_freq(500000.0, 128)
    np.testing.assert_allclose(oracle_mod.rope_inv_freq(500000.0, 128, factors), base / factors, rtol=1e-6)


def _rope_f64(x, n_heads, hd, pos, inv_freq):
    """Textbook rotation of pairs (2i, 2i+1) in float64, by the angle the reference forms in
    float32: float(pos) * inv_freq[i] (src/ops.cpp:248), rounded once."""
    x = np.asarray(x, dtype=np.float64).reshape(x.shape[0], n_heads, hd // 2, 2).copy()
    p32 = (pos + np.arange(x.shape[0])).astype(np.float32)
    ang = (p32[:, None] * inv_freq.astype(np.float32)[None, :]).astype(np.float64)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x0, x1 = x[..., 0].copy(), x[..., 1].copy()
    x[..., 0] = x0 * c - x1 * s
    x[..., 1] = x0 * s + x1 * c
    return x.reshape(x.shape[0], -1)


def test_rope_pins(oracle_mod):
    rng = np.random.default_rng(3)
    inv = oracle_mod.rope_inv_freq(500000.0, 128)
    x = rng.standard_normal((6, 3 * 128)).astype(np.float32)
    # position 0 is the identity (cos 0 = 1, sin 0 = 0 exactly)
    assert np.array_equal(oracle_mod.rope(x[:1], 3, 128, 0, inv), x[:1])
    # the textbook rotation of adjacent pairs, in float64 (pins pair layout, sign, angle)
    for pos in (1, 17, 4000):
        got = oracle_mod.rope(x, 3, 128, pos, inv)
        np.testing.assert_allclose(got, _rope_f64(x, 3, 128, pos, inv), rtol=0, atol=2e-6)
    # a rotation keeps every pair's length
    got = oracle_mod.rope(x, 3, 128, 123, inv).reshape(6, -1, 2)
    np.testing.assert_allclose(np.hypot(got[..., 0], got[..., 1]),
                               np.hypot(*x.reshape(6, -1, 2).transpose(2, 0, 1)), rtol=1e-5)


def test_kv_store_is_rope_then_f16(oracle_mod):
    rng = np.random.default_rng(5)
    hkv, hd, n_tok, pos, n_ctx = 2, 128, 5, 7, 16
    inv = oracle_mod.rope_inv_freq(10000.0, hd)
    k = rng.standard_normal((n_tok, hkv * hd)).astype(np.float32)
    v = rng.standard_normal((n_tok, hkv * hd)).astype(np.float32)
    q = rng.standard_normal((n_tok, 4 * hd)).astype(np.float32)
    canary = np.full((2 * n_ctx, hkv * hd), 0x7E00, dtype=np.uint16)
    dst = (n_ctx + pos) * hkv * hd  # layer 1
    qq, kc, vc = oracle_mod.rope_kv_store(q, k, v, canary, canary, dst, 4, hkv, hd, pos, inv)
    rows = slice(n_ctx + pos, n_ctx + pos + n_tok)
    assert np.array_equal(vc[rows], oracle_mod.f32_to_f16(v))
    assert np.array_equal(kc[rows], oracle_mod.f32_to_f16(oracle_mod.rope(k, hkv, hd, pos, inv)))
    np.testing.assert_array_equal(qq, oracle_mod.rope(q, 4, hd, pos, inv))
    others = np.ones(2 * n_ctx, dtype=bool)
    others[rows] = False
    assert (kc[others] == 0x7E00).all() and (vc[others] == 0x7E00).all()
