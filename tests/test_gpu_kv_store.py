"""GPU parity of the fused RoPE + KV-cache store (ingot_rope_kv_store) against the CPU oracle.

Tolerances, stated per output:
  - V in the cache: bit-exact (a pure f32 -> f16 round-to-nearest-even conversion);
  - K in the cache: the GPU's sincosf and the host's cosf/sinf may differ in the last f32 bit,
    and the products may be fused on the GPU, so an element whose rotated value sits next to an
    f16 rounding tie can land one f16 step away: |d| <= 1 f16 ulp everywhere, and >= 99.5% of
    the elements bit-exact;
  - q rotated in place (f32): |d| <= 2e-6 * (1 + |q|) per element;
  - rows of the cache outside the written ones keep their (NaN) canary bits;
  - end to end, attention over the GPU-written cache with the GPU-rotated q matches the oracle's
    rope + store + attention within the attention tolerance (max|d| 2e-3, rel-L2 1e-3).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_parity, ensure_built

pytestmark = pytest.mark.gpu

H, HKV, HD = 24, 8, 128
KV = HKV * HD
THETA = 500000.0


@pytest.fixture(scope="module")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a GPU")
    ensure_built("lib")
    import ingot_attn

    ingot_attn.load_library()
    return torch.device("cuda:0")


def _t(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _llama3_factors():
    """Per-frequency divisors of the kind Llama 3.1+ GGUFs carry in rope_freqs.weight."""
    f = np.ones(HD // 2, dtype=np.float32)
    f[HD // 4:] = np.linspace(1.0, 8.0, HD // 4, dtype=np.float32)
    return f


def _f16_ulps(a_bits, b_bits):
    """Distance in f16 steps between two arrays of finite f16 bit patterns."""
    def key(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(key(a_bits) - key(b_bits))


def _run(dev, oracle_mod, seed, pos, n_tok, with_q=True, layer=1, n_ctx=None, kv_pad=0, q_pad=0):
    import torch
    import ingot_attn as ia

    n_ctx = pos + n_tok + 3 if n_ctx is None else n_ctx
    print(f"[rope_kv_store] seed={seed} pos={pos} n_tok={n_tok} q={with_q} layer={layer} "
          f"n_ctx={n_ctx} kv_pad={kv_pad} q_pad={q_pad}", flush=True)
    rng = np.random.default_rng(seed)
    inv = oracle_mod.rope_inv_freq(THETA, HD, _llama3_factors())
    k = rng.standard_normal((n_tok, KV + kv_pad)).astype(np.float32)
    v = rng.standard_normal((n_tok, KV + kv_pad)).astype(np.float32)
    q = rng.standard_normal((n_tok, H * HD + q_pad)).astype(np.float32)
    cache = np.full(((layer + 1) * n_ctx, KV), 0x7E00, dtype=np.uint16)
    dst = (layer * n_ctx + pos) * KV
    qo, kc_want, vc_want = oracle_mod.rope_kv_store(q[:, :H * HD] if with_q else None, k, v, cache,
                                                    cache, dst, H, HKV, HD, pos, inv)
    qd = _t(q, dev)
    kd, vd = _t(k, dev), _t(v, dev)
    kcd = _t(cache.view(np.int16), dev)
    vcd = _t(cache.view(np.int16), dev)
    desc = ia.rope_kv_desc(H, HKV, HD, pos, n_tok, dst_offset=dst, q_stride=H * HD + q_pad,
                           kv_stride=KV + kv_pad)
    ia.rope_kv_store(qd if with_q else None, kd, vd, kcd, vcd, _t(inv, dev), desc)
    torch.cuda.synchronize()
    return (qd.cpu().numpy(), q, qo, kcd.cpu().numpy().view(np.uint16), kc_want,
            vcd.cpu().numpy().view(np.uint16), vc_want, dst // KV, n_tok)


def _check(res):
    q_got, q_in, q_want, kc, kc_want, vc, vc_want, row0, n_tok = res
    rows = slice(row0, row0 + n_tok)
    assert np.array_equal(vc, vc_want), "V cache rows differ (must be bit-exact)"
    ulps = _f16_ulps(kc[rows], kc_want[rows])
    exact = float((ulps == 0).mean())
    print(f"K: max {int(ulps.max())} f16 ulp, {100 * exact:.3f}% bit-exact", flush=True)
    assert ulps.max() <= 1 and exact >= 0.995
    others = np.ones(kc.shape[0], dtype=bool)
    others[rows] = False
    assert (kc[others] == 0x7E00).all() and (vc[others] == 0x7E00).all(), "rows outside were written"
    if q_want is not None:
        w = q_want.shape[1]
        tol = 2e-6 * (1 + np.abs(q_want))
        d = np.abs(q_got[:, :w] - q_want)
        assert (d <= tol).all(), f"q max|d| {d.max():.3e}"
        assert np.array_equal(q_got[:, w:], q_in[:, w:]), "q row padding changed"
    else:
        assert np.array_equal(q_got, q_in), "q changed although it was not passed"


@pytest.mark.parametrize("pos,n_tok", [(0, 1), (5, 1), (4095, 1), (0, 7), (3584, 512), (8000, 33)])
def test_rope_kv_store_parity(dev, oracle_mod, pos, n_tok):
    _check(_run(dev, oracle_mod, 11 + pos + n_tok, pos, n_tok))


def test_rope_kv_store_without_q(dev, oracle_mod):
    _check(_run(dev, oracle_mod, 5, 100, 9, with_q=False))


def test_rope_kv_store_padded_strides_and_layer(dev, oracle_mod):
    _check(_run(dev, oracle_mod, 6, 40, 17, layer=3, kv_pad=64, q_pad=128))


def test_store_then_attention_end_to_end(dev, oracle_mod):
    """Decode and prefill over a cache written by ingot_rope_kv_store vs the oracle pipeline."""
    import torch
    import ingot_attn as ia

    rng = np.random.default_rng(99)
    inv = oracle_mod.rope_inv_freq(THETA, HD, _llama3_factors())
    n_ctx, pos, n_tok = 700, 600, 64
    # prefix rows 0..pos-1 exist already; the chunk pos..pos+n_tok-1 is stored now
    prefix_k = (rng.standard_normal((pos, KV))).astype(np.float16).view(np.uint16)
    prefix_v = (rng.standard_normal((pos, KV))).astype(np.float16).view(np.uint16)
    kc0 = np.full((n_ctx, KV), 0x7E00, dtype=np.uint16)
    vc0 = kc0.copy()
    kc0[:pos], vc0[:pos] = prefix_k, prefix_v
    k = rng.standard_normal((n_tok, KV)).astype(np.float32)
    v = rng.standard_normal((n_tok, KV)).astype(np.float32)
    q = rng.standard_normal((n_tok, H * HD)).astype(np.float32)
    q_w, kc_w, vc_w = oracle_mod.rope_kv_store(q, k, v, kc0, vc0, pos * KV, H, HKV, HD, pos, inv)
    want = oracle_mod.attn_prefill(q_w, kc_w, vc_w, H, HKV, HD, pos, n_tok, threads=8)

    qd, kd, vd = _t(q, dev), _t(k, dev), _t(v, dev)
    kcd, vcd = _t(kc0.view(np.int16), dev), _t(vc0.view(np.int16), dev)
    ia.rope_kv_store(qd, kd, vd, kcd, vcd, _t(inv, dev), ia.rope_kv_desc(H, HKV, HD, pos, n_tok, dst_offset=pos * KV))
    out = torch.full_like(qd, float("nan"))
    ia.attn_prefill(qd, kcd, vcd, out, ia.prefill_desc(H, HKV, HD, pos, n_tok))
    torch.cuda.synchronize()
    assert_parity(out.cpu().numpy(), want, "prefill over the stored cache")
    # the last token as a decode step
    outd = torch.full((H * HD,), float("nan"), device=dev)
    ia.attn_decode(qd[-1].contiguous(), kcd, vcd, outd, ia.decode_desc(H, HKV, HD, pos + n_tok))
    torch.cuda.synchronize()
    assert_parity(outd.cpu().numpy(), want[-1], "decode over the stored cache")


@pytest.mark.parametrize("n_head,n_head_kv,hd", [(8, 8, 128), (16, 4, 128), (3, 1, 128), (32, 8, 64), (4, 2, 256)])
def test_rope_kv_store_shapes(dev, oracle_mod, n_head, n_head_kv, hd):
    """Other head counts and head sizes (the store itself is not limited to head_dim 128)."""
    import torch
    import ingot_attn as ia

    print(f"[rope_kv_store shapes] H={n_head} HKV={n_head_kv} hd={hd}", flush=True)
    rng = np.random.default_rng(n_head * 31 + hd)
    pos, n_tok, n_ctx = 123, 9, 140
    kv = n_head_kv * hd
    inv = oracle_mod.rope_inv_freq(10000.0, hd)
    q = rng.standard_normal((n_tok, n_head * hd)).astype(np.float32)
    k = rng.standard_normal((n_tok, kv)).astype(np.float32)
    v = rng.standard_normal((n_tok, kv)).astype(np.float32)
    cache = np.full((n_ctx, kv), 0x7E00, dtype=np.uint16)
    q_w, kc_w, vc_w = oracle_mod.rope_kv_store(q, k, v, cache, cache, pos * kv, n_head, n_head_kv, hd, pos, inv)
    qd = _t(q, dev)
    kcd, vcd = _t(cache.view(np.int16), dev), _t(cache.view(np.int16), dev)
    ia.rope_kv_store(qd, _t(k, dev), _t(v, dev), kcd, vcd, _t(inv, dev),
                     ia.rope_kv_desc(n_head, n_head_kv, hd, pos, n_tok, dst_offset=pos * kv))
    torch.cuda.synchronize()
    _check((qd.cpu().numpy(), q, q_w, kcd.cpu().numpy().view(np.uint16), kc_w,
            vcd.cpu().numpy().view(np.uint16), vc_w, pos, n_tok))
