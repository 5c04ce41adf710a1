"""GPU parity of the causal MFMA prefill kernel against the CPU oracle, through the C ABI."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_parity, ensure_built

pytestmark = pytest.mark.gpu

H, HKV, HD = 24, 8, 128
KV = HKV * HD


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


def _run_prefill(dev, q, kb, vb, n_head, n_head_kv, pos, n_tok, kv_offset=0, n_splits=0,
                 q_stride=None, head_dim=HD):
    import torch
    import ingot_attn as ia

    q_stride = n_head * head_dim if q_stride is None else q_stride
    print(f"[prefill] n_head={n_head} n_head_kv={n_head_kv} pos={pos} n_tok={n_tok} "
          f"kv_offset={kv_offset} n_splits={n_splits} q_stride={q_stride}", flush=True)
    qd = _t(q.astype(np.float32), dev)
    kd = _t(kb.view(np.int16), dev)
    vd = _t(vb.view(np.int16), dev)
    out = torch.full(qd.shape, float("nan"), dtype=torch.float32, device=dev)
    desc = ia.prefill_desc(n_head, n_head_kv, head_dim, pos, n_tok, kv_offset=kv_offset,
                           q_stride=q_stride, n_splits=n_splits)
    ia.attn_prefill(qd, kd, vd, out, desc)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _inputs(seed, n_head, n_head_kv, pos, n_tok, n_ctx=None):
    rng = np.random.Generator(np.random.PCG64(seed))
    L = pos + n_tok
    n_ctx = L if n_ctx is None else n_ctx
    q = rng.standard_normal((n_tok, n_head * HD)).astype(np.float32)
    kb = np.full((n_ctx, n_head_kv * HD), 0x7E00, dtype=np.uint16)
    vb = np.full((n_ctx, n_head_kv * HD), 0x7E00, dtype=np.uint16)
    kb[:L] = rng.standard_normal((L, n_head_kv * HD)).astype(np.float16).view(np.uint16)
    vb[:L] = rng.standard_normal((L, n_head_kv * HD)).astype(np.float16).view(np.uint16)
    return q, kb, vb


@pytest.mark.parametrize("name", ["C2-prefill-512@0", "C4-prefill-512@3584"])
def test_prefill_configs(dev, oracle_mod, name):
    import workloads as W

    w = W.BY_NAME[name]
    q, kb, vb = W.make_inputs(w)
    got = _run_prefill(dev, q, kb, vb, H, HKV, w.pos, w.n_tok)
    want = oracle_mod.attn_prefill(q, kb, vb, H, HKV, HD, w.pos, w.n_tok, threads=16)
    m, r = assert_parity(got, want, name)
    print(f"{name}: max|d|={m:.2e} rel-L2={r:.2e}")


def test_prefill_c5_full(dev, oracle_mod):
    # C5's prefill in full: 2048 queries at 6144 over 8192 keys, every row and head against the
    # oracle (about 25 s of CPU on 16 threads).
    import os

    import workloads as W

    w = W.C5_PREFILL
    q, kb, vb = W.make_inputs(w)
    got = _run_prefill(dev, q, kb, vb, H, HKV, w.pos, w.n_tok)
    want = oracle_mod.attn_prefill(q, kb, vb, H, HKV, HD, w.pos, w.n_tok, threads=min(16, os.cpu_count() or 1))
    m, r = assert_parity(got, want, "C5 prefill (all 2048 rows)")
    print(f"C5 prefill full: max|d|={m:.2e} rel-L2={r:.2e}")


@pytest.mark.parametrize("pos,n_tok", [(0, 1), (0, 2), (0, 7), (0, 33), (5, 64), (100, 65),
                                       (63, 1), (64, 31), (1000, 97), (0, 160),
                                       # either side of the one-workgroup-per-query-head limit
                                       # (query blocks x 24 heads <= 256): 240 and 264
                                       (0, 640), (0, 704)])
def test_prefill_ragged(dev, oracle_mod, pos, n_tok):
    q, kb, vb = _inputs(pos * 7 + n_tok, H, HKV, pos, n_tok, n_ctx=pos + n_tok + 70)
    got = _run_prefill(dev, q, kb, vb, H, HKV, pos, n_tok)
    want = oracle_mod.attn_prefill(q, kb, vb, H, HKV, HD, pos, n_tok, threads=8)
    assert_parity(got, want, f"pos={pos} n_tok={n_tok}")


@pytest.mark.parametrize("splits", [1, 2, 3, 5, 16])
def test_prefill_split_invariance(dev, oracle_mod, splits):
    pos, n_tok = 900, 100
    q, kb, vb = _inputs(31, H, HKV, pos, n_tok)
    got = _run_prefill(dev, q, kb, vb, H, HKV, pos, n_tok, n_splits=splits)
    want = oracle_mod.attn_prefill(q, kb, vb, H, HKV, HD, pos, n_tok, threads=8)
    assert_parity(got, want, f"splits={splits}")


@pytest.mark.parametrize("n_head,n_head_kv", [(8, 8), (8, 4), (16, 4), (3, 1)])
def test_prefill_group_sizes(dev, oracle_mod, n_head, n_head_kv):
    pos, n_tok = 70, 90
    q, kb, vb = _inputs(n_head, n_head, n_head_kv, pos, n_tok)
    got = _run_prefill(dev, q, kb, vb, n_head, n_head_kv, pos, n_tok)
    want = oracle_mod.attn_prefill(q, kb, vb, n_head, n_head_kv, HD, pos, n_tok)
    assert_parity(got, want, f"G={n_head // n_head_kv}")


@pytest.mark.parametrize("n_head,n_head_kv,n_tok", [(64, 32, 300), (48, 16, 400), (64, 16, 300)])
def test_prefill_group_sizes_whole_groups(dev, oracle_mod, n_head, n_head_kv, n_tok):
    """Chunks whose query blocks x query heads exceed the 256 CUs keep a group's heads in one
    workgroup (the chunks above run one workgroup per query head): G = 2, 3, 4, unsplit."""
    pos = 40
    q, kb, vb = _inputs(n_head + n_tok, n_head, n_head_kv, pos, n_tok)
    got = _run_prefill(dev, q, kb, vb, n_head, n_head_kv, pos, n_tok, n_splits=1)
    want = oracle_mod.attn_prefill(q, kb, vb, n_head, n_head_kv, HD, pos, n_tok, threads=8)
    assert_parity(got, want, f"G={n_head // n_head_kv} whole groups")


def test_prefill_layer_offset_and_stride(dev, oracle_mod):
    # layer slice 1 of a 3-layer cache (other layers NaN) and a padded q/out row stride
    n_ctx, pos, n_tok = 300, 150, 77
    q, kb1, vb1 = _inputs(42, H, HKV, pos, n_tok, n_ctx=n_ctx)
    kb = np.full((3 * n_ctx, KV), 0x7E00, dtype=np.uint16)
    vb = np.full((3 * n_ctx, KV), 0x7E00, dtype=np.uint16)
    kb[n_ctx:2 * n_ctx] = kb1
    vb[n_ctx:2 * n_ctx] = vb1
    stride = H * HD + 64
    qp = np.zeros((n_tok, stride), dtype=np.float32)
    qp[:, : H * HD] = q
    got = _run_prefill(dev, qp, kb, vb, H, HKV, pos, n_tok, kv_offset=n_ctx * KV, q_stride=stride)
    want = oracle_mod.attn_prefill(q, kb1, vb1, H, HKV, HD, pos, n_tok)
    assert_parity(got[:, : H * HD], want, "offset+stride")
    assert np.all(np.isnan(got[:, H * HD:])), "wrote outside the heads' columns"


def test_prefill_rows_equal_decode_steps(dev):
    # Property that holds at any size: prefill row i == decode with n_keys = pos+i+1 (both GPU).
    import torch
    import ingot_attn as ia

    pos, n_tok = 2000, 96
    q, kb, vb = _inputs(55, H, HKV, pos, n_tok)
    got = _run_prefill(dev, q, kb, vb, H, HKV, pos, n_tok)
    kd, vd = _t(kb.view(np.int16), dev), _t(vb.view(np.int16), dev)
    for i in (0, 17, 95):
        out = torch.empty(H * HD, dtype=torch.float32, device=dev)
        ia.attn_decode(_t(q[i], dev), kd, vd, out, ia.decode_desc(H, HKV, HD, pos + i + 1))
        torch.cuda.synchronize()
        assert_parity(got[i], out.cpu().numpy(), f"row {i}")


@pytest.mark.parametrize("n_head,n_head_kv,hd", [(32, 8, 64), (16, 8, 256), (64, 8, 128), (48, 8, 128),
                                                  (40, 8, 128), (16, 2, 64)])
def test_prefill_head_dims_and_groups(dev, oracle_mod, n_head, n_head_kv, hd):
    # head_dim 64 and 256 and groups above 3 on the MFMA kernel (units of up to 3 heads, 1 for
    # head_dim 256): the reference takes these through its flash prefill (any group,
    # src/metal_backend.mm:360) or its naive kernel (shaders/kernels.metal:639-702).
    import ingot_attn as ia
    import torch

    pos, n_tok = 40, 300
    rng = np.random.Generator(np.random.PCG64(n_head * hd))
    L = pos + n_tok
    q = rng.standard_normal((n_tok, n_head * hd)).astype(np.float32)
    kb = rng.standard_normal((L, n_head_kv * hd)).astype(np.float16).view(np.uint16)
    vb = rng.standard_normal((L, n_head_kv * hd)).astype(np.float16).view(np.uint16)
    print(f"[prefill] n_head={n_head} n_head_kv={n_head_kv} hd={hd} {n_tok}@{pos}", flush=True)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    out = torch.full((n_tok, n_head * hd), float("nan"), device=dev)
    ia.attn_prefill(t(q), t(kb.view(np.int16)), t(vb.view(np.int16)), out,
                    ia.prefill_desc(n_head, n_head_kv, hd, pos, n_tok))
    torch.cuda.synchronize()
    want = oracle_mod.attn_prefill(q, kb, vb, n_head, n_head_kv, hd, pos, n_tok, threads=8)
    assert_parity(out.cpu().numpy(), want, f"prefill hd={hd} G={n_head // n_head_kv}")


def test_prefill_group8_split(dev, oracle_mod):
    # G = 8 with the key range split (a long chunk over a long prefix)
    import ingot_attn as ia
    import torch

    n_head, n_head_kv, pos, n_tok = 64, 8, 3000, 512
    d = ia.prefill_desc(n_head, n_head_kv, 128, pos, n_tok)
    print(f"[prefill] G=8 {n_tok}@{pos} splits={ia.prefill_splits(d)}", flush=True)
    q, kb, vb = _inputs(88, n_head, n_head_kv, pos, n_tok)
    got = _run_prefill(dev, q, kb, vb, n_head, n_head_kv, pos, n_tok)
    want = oracle_mod.attn_prefill(q, kb, vb, n_head, n_head_kv, 128, pos, n_tok, threads=16)
    assert_parity(got, want, "prefill G=8 split")


@pytest.mark.parametrize("hd,n_head,n_head_kv,pos,n_tok", [
    (64, 32, 8, 3000, 512), (64, 24, 8, 0, 512), (64, 16, 2, 1000, 130),
    (256, 16, 8, 3000, 512), (256, 16, 8, 0, 256), (256, 12, 4, 700, 77)])
def test_prefill_mfma_head_dims(dev, oracle_mod, hd, n_head, n_head_kv, pos, n_tok):
    # head_dim 64 and 256 on the MFMA kernel: a long prefix (key split + combine), a chunk from 0
    # (the head split), and a ragged chunk with few KV heads.
    import ingot_attn as ia

    d = ia.prefill_desc(n_head, n_head_kv, hd, pos, n_tok)
    print(f"[prefill] hd={hd} {n_head}/{n_head_kv} {n_tok}@{pos} splits={ia.prefill_splits(d)}", flush=True)
    rng = np.random.Generator(np.random.PCG64(7 * n_head + pos + hd))
    L = pos + n_tok
    q = rng.standard_normal((n_tok, n_head * hd)).astype(np.float32)
    kb = rng.standard_normal((L, n_head_kv * hd)).astype(np.float16).view(np.uint16)
    vb = rng.standard_normal((L, n_head_kv * hd)).astype(np.float16).view(np.uint16)
    got = _run_prefill(dev, q, kb, vb, n_head, n_head_kv, pos, n_tok, head_dim=hd)
    want = oracle_mod.attn_prefill(q, kb, vb, n_head, n_head_kv, hd, pos, n_tok, threads=16)
    assert_parity(got, want, f"prefill hd={hd} {n_head}/{n_head_kv} {n_tok}@{pos}")


@pytest.mark.parametrize("hd,n_head,n_head_kv,pos,n_tok", [
    (80, 32, 8, 0, 70), (96, 24, 8, 1000, 37), (112, 12, 4, 300, 5), (160, 8, 2, 0, 300),
    (20, 4, 4, 17, 9), (1024, 2, 1, 260, 3), (3, 6, 3, 0, 40), (96, 8, 2, 3000, 1),
    # blocks of 8 tokens (keys beyond one chunk): odd and 2-aligned rows, 1, 2 and 4 dim groups
    # per thread
    (3, 6, 3, 500, 20), (1023, 2, 1, 300, 9), (1022, 2, 1, 280, 10), (510, 4, 2, 700, 17)])
def test_prefill_fallback_head_dims(dev, oracle_mod, hd, n_head, n_head_kv, pos, n_tok):
    # Head sizes without an MFMA kernel run the fallback kernel, the counterpart of the
    # reference's naive attention (shaders/kernels.metal:639-702, chosen at
    # src/metal_backend.mm:373-382 for every head_dim but 128).
    import ingot_attn as ia

    d = ia.prefill_desc(n_head, n_head_kv, hd, pos, n_tok)
    assert ia.prefill_splits(d) == 1
    rng = np.random.Generator(np.random.PCG64(11 * n_head + pos + hd))
    L = pos + n_tok
    q = rng.standard_normal((n_tok, n_head * hd)).astype(np.float32)
    kb = np.full((L + 5, n_head_kv * hd), 0x7E00, dtype=np.uint16)  # NaN past the chunk
    vb = np.full((L + 5, n_head_kv * hd), 0x7E00, dtype=np.uint16)
    kb[:L] = rng.standard_normal((L, n_head_kv * hd)).astype(np.float16).view(np.uint16)
    vb[:L] = rng.standard_normal((L, n_head_kv * hd)).astype(np.float16).view(np.uint16)
    got = _run_prefill(dev, q, kb, vb, n_head, n_head_kv, pos, n_tok, head_dim=hd)
    want = oracle_mod.attn_prefill(q, kb, vb, n_head, n_head_kv, hd, pos, n_tok, threads=8)
    assert_parity(got, want, f"fallback prefill hd={hd} {n_head}/{n_head_kv} {n_tok}@{pos}")
