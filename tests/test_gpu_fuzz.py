"""Seeded random sweeps of decode and prefill shapes through the C ABI against the CPU oracle:
head size (the MFMA sizes 64/128/256 and odd sizes for the fallback kernel), group size, cache
length, chunk position and length, forced or library-chosen splits, a layer offset into a
multi-layer cache, a padded q_stride and the descriptor's scale — combinations the hand-picked cases do not reach.
Every case prints its parameters before the GPU call. Bar: max|d| <= 2e-3, rel-L2 <= 1e-3."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_parity, ensure_built

pytestmark = pytest.mark.gpu

HEAD_DIMS = [64, 128, 128, 128, 256, 96, 80, 40, 18]
GROUPS = [(8, 8), (16, 8), (24, 8), (32, 8), (12, 4), (40, 8), (64, 8), (6, 2), (4, 1), (48, 8), (96, 8)]


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


def _cache(rng, n_layer, n_ctx, kv_dim, L, layer):
    kb = np.full((n_layer * n_ctx, kv_dim), 0x7E00, dtype=np.uint16)  # NaN outside the slice
    vb = np.full((n_layer * n_ctx, kv_dim), 0x7E00, dtype=np.uint16)
    r0 = layer * n_ctx
    kb[r0:r0 + L] = rng.standard_normal((L, kv_dim)).astype(np.float16).view(np.uint16)
    vb[r0:r0 + L] = rng.standard_normal((L, kv_dim)).astype(np.float16).view(np.uint16)
    return kb, vb


@pytest.mark.parametrize("case", range(48))
def test_decode_random_shapes(dev, oracle_mod, case):
    import torch
    import ingot_attn as ia

    rng = np.random.Generator(np.random.PCG64(1000 + case))
    hd = int(rng.choice(HEAD_DIMS))
    n_head, n_head_kv = GROUPS[int(rng.integers(len(GROUPS)))]
    L = int(rng.choice([1, 2, 17, 100, 193, 511, 1000, 2500, 4100]))
    splits = int(rng.choice([0, 0, 0, 1, 3, 8, 32]))
    n_layer, layer = 3, int(rng.integers(3))
    n_ctx = L + int(rng.integers(0, 40))
    kv_dim = n_head_kv * hd
    scale = None if case % 3 else float(rng.choice([0.02, 0.3, 1.0]))  # the descriptor's own scale
    print(f"[fuzz decode {case}] {n_head}/{n_head_kv} hd={hd} L={L} splits={splits} layer={layer} "
          f"n_ctx={n_ctx} scale={scale}", flush=True)
    kb, vb = _cache(rng, n_layer, n_ctx, kv_dim, L, layer)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    out = torch.full((n_head * hd,), float("nan"), dtype=torch.float32, device=dev)
    desc = ia.decode_desc(n_head, n_head_kv, hd, L, kv_offset=layer * n_ctx * kv_dim, n_splits=splits, scale=scale)
    ia.attn_decode(_t(q, dev), _t(kb.view(np.int16), dev), _t(vb.view(np.int16), dev), out, desc)
    torch.cuda.synchronize()
    r0 = layer * n_ctx
    want = oracle_mod.attn_decode(q, kb[r0:r0 + L], vb[r0:r0 + L], n_head, n_head_kv, hd, L, scale=scale, threads=8)
    assert_parity(out.cpu().numpy(), want, f"decode case {case}")


@pytest.mark.parametrize("case", range(40))
def test_prefill_random_shapes(dev, oracle_mod, case):
    import torch
    import ingot_attn as ia

    rng = np.random.Generator(np.random.PCG64(2000 + case))
    hd = int(rng.choice(HEAD_DIMS))
    n_head, n_head_kv = GROUPS[int(rng.integers(len(GROUPS)))]
    pos = int(rng.choice([0, 0, 5, 64, 300, 1000, 2000]))
    n_tok = int(rng.choice([2, 9, 64, 65, 130, 257]))
    splits = int(rng.choice([0, 0, 0, 1, 2, 5]))
    L = pos + n_tok
    n_layer, layer = 2, int(rng.integers(2))
    n_ctx = L + int(rng.integers(0, 20))
    kv_dim = n_head_kv * hd
    pad = int(rng.choice([0, 0, 4, 36]))  # q_stride padding (a multiple of 4)
    q_stride = n_head * hd + pad
    # (the MFMA prefill rounds q * scale to f16, as the reference's GPU path does, so the score
    # error grows with the scale: scales of the size attention uses, around 1/sqrt(head_dim))
    scale = None if case % 3 else float(rng.choice([0.02, 0.06, 0.12]))
    print(f"[fuzz prefill {case}] {n_head}/{n_head_kv} hd={hd} pos={pos} n_tok={n_tok} splits={splits} "
          f"layer={layer} q_stride={q_stride} scale={scale}", flush=True)
    kb, vb = _cache(rng, n_layer, n_ctx, kv_dim, L, layer)
    qf = np.full((n_tok, q_stride), np.nan, dtype=np.float32)
    qf[:, :n_head * hd] = rng.standard_normal((n_tok, n_head * hd)).astype(np.float32)
    out = torch.full((n_tok, q_stride), float("nan"), dtype=torch.float32, device=dev)
    desc = ia.prefill_desc(n_head, n_head_kv, hd, pos, n_tok, kv_offset=layer * n_ctx * kv_dim,
                           q_stride=q_stride, n_splits=splits, scale=scale)
    ia.attn_prefill(_t(qf, dev), _t(kb.view(np.int16), dev), _t(vb.view(np.int16), dev), out, desc)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    r0 = layer * n_ctx
    want = oracle_mod.attn_prefill(qf[:, :n_head * hd], kb[r0:r0 + L], vb[r0:r0 + L], n_head, n_head_kv, hd,
                                   pos, n_tok, scale=scale, threads=8)
    assert_parity(got[:, :n_head * hd], want.reshape(n_tok, -1), f"prefill case {case}")
    if pad:
        assert np.isnan(got[:, n_head * hd:]).all(), "the padding columns of out were written"
