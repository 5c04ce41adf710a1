"""GPU parity of the split-KV decode kernel against the CPU oracle, through the C ABI."""
from __future__ import annotations

import math
import sys

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


def _run_decode(dev, q, kb, vb, n_head, n_head_kv, n_keys, kv_offset=0, n_splits=0, hd=HD,
                workspace=None):
    import torch
    import ingot_attn as ia

    print(f"[decode] n_head={n_head} n_head_kv={n_head_kv} hd={hd} n_keys={n_keys} "
          f"kv_offset={kv_offset} n_splits={n_splits}", flush=True)
    qd = _t(q.astype(np.float32), dev)
    kd = _t(kb.view(np.int16), dev)
    vd = _t(vb.view(np.int16), dev)
    out = torch.full((n_head * hd,), float("nan"), dtype=torch.float32, device=dev)
    desc = ia.decode_desc(n_head, n_head_kv, hd, n_keys, kv_offset=kv_offset, n_splits=n_splits)
    ia.attn_decode(qd, kd, vd, out, desc, workspace=workspace)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _inputs(seed, n_head, n_head_kv, L, kv_scale=1.0, n_ctx=None, hd=HD):
    rng = np.random.Generator(np.random.PCG64(seed))
    n_ctx = L if n_ctx is None else n_ctx
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    kb = np.full((n_ctx, n_head_kv * hd), 0x7E00, dtype=np.uint16)  # NaN past n_keys
    vb = np.full((n_ctx, n_head_kv * hd), 0x7E00, dtype=np.uint16)
    kb[:L] = (rng.standard_normal((L, n_head_kv * hd)) * kv_scale).astype(np.float16).view(np.uint16)
    vb[:L] = (rng.standard_normal((L, n_head_kv * hd)) * kv_scale).astype(np.float16).view(np.uint16)
    return q, kb, vb


@pytest.mark.parametrize("name", ["C1-decode-512", "C3-decode-4096", "C5-decode-1024",
                                  "C5-decode-2048", "C5-decode-4096", "C5-decode-8192"])
def test_decode_configs(dev, oracle_mod, name):
    import workloads as W

    w = W.BY_NAME[name]
    q, kb, vb = W.make_inputs(w)
    got = _run_decode(dev, q, kb, vb, H, HKV, w.n_keys)
    want = oracle_mod.attn_decode(q, kb, vb, H, HKV, HD, w.n_keys, threads=8)
    m, r = assert_parity(got, want, name)
    print(f"{name}: max|d|={m:.2e} rel-L2={r:.2e}")


@pytest.mark.parametrize("L", [1, 2, 3, 15, 16, 17, 63, 64, 65, 100, 127, 129, 1000, 4097])
def test_decode_ragged_lengths(dev, oracle_mod, L):
    q, kb, vb = _inputs(1000 + L, H, HKV, L, n_ctx=L + 40)
    got = _run_decode(dev, q, kb, vb, H, HKV, L)
    want = oracle_mod.attn_decode(q, kb, vb, H, HKV, HD, L)
    assert_parity(got, want, f"L={L}")


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 33, 48, 64, 200, 1024])
def test_decode_split_invariance(dev, oracle_mod, splits):
    L = 2000
    q, kb, vb = _inputs(77, H, HKV, L)
    got = _run_decode(dev, q, kb, vb, H, HKV, L, n_splits=splits)
    want = oracle_mod.attn_decode(q, kb, vb, H, HKV, HD, L)
    assert_parity(got, want, f"splits={splits}")


@pytest.mark.parametrize("n_head,n_head_kv", [(8, 8), (8, 4), (16, 4), (32, 8), (3, 1)])
def test_decode_group_sizes(dev, oracle_mod, n_head, n_head_kv):
    L = 333
    q, kb, vb = _inputs(5 + n_head, n_head, n_head_kv, L)
    got = _run_decode(dev, q, kb, vb, n_head, n_head_kv, L)
    want = oracle_mod.attn_decode(q, kb, vb, n_head, n_head_kv, HD, L)
    assert_parity(got, want, f"G={n_head // n_head_kv}")


def test_decode_layer_offset(dev, oracle_mod):
    # A 4-layer cache [layer][n_ctx][kv_dim]; layers other than 2 hold NaN, so reading outside
    # the selected slice shows up as a non-finite output.
    n_ctx, L, layer = 600, 517, 2
    q, kb1, vb1 = _inputs(9, H, HKV, L, n_ctx=n_ctx)
    kb = np.full((4 * n_ctx, KV), 0x7E00, dtype=np.uint16)
    vb = np.full((4 * n_ctx, KV), 0x7E00, dtype=np.uint16)
    kb[layer * n_ctx:(layer + 1) * n_ctx] = kb1
    vb[layer * n_ctx:(layer + 1) * n_ctx] = vb1
    got = _run_decode(dev, q, kb, vb, H, HKV, L, kv_offset=layer * n_ctx * KV)
    want = oracle_mod.attn_decode(q, kb1, vb1, H, HKV, HD, L)
    assert_parity(got, want, "layer offset")


def test_decode_repeated_calls_reuse_workspace(dev, oracle_mod):
    # Every call leaves its counters and records at zero, so the next one starts clean.
    for i, L in enumerate((4096, 700, 4096, 65)):
        q, kb, vb = _inputs(300 + i, H, HKV, L)
        got = _run_decode(dev, q, kb, vb, H, HKV, L)
        want = oracle_mod.attn_decode(q, kb, vb, H, HKV, HD, L, threads=8)
        assert_parity(got, want, f"call {i}")


@pytest.mark.parametrize("n_head,n_head_kv,hd", [(32, 8, 64), (16, 8, 256), (8, 8, 64), (4, 2, 256)])
@pytest.mark.parametrize("L", [1, 513, 4097])
def test_decode_head_dims(dev, oracle_mod, n_head, n_head_kv, hd, L):
    # Llama-3.2-1B (32 Q / 8 KV, head_dim 64) and a head_dim-256 model; the reference serves
    # these through its naive kernel (src/metal_backend.mm:373-382, shaders/kernels.metal:639-702).
    q, kb, vb = _inputs(40 + L + hd, n_head, n_head_kv, L, n_ctx=L + 8, hd=hd)
    got = _run_decode(dev, q, kb, vb, n_head, n_head_kv, L, hd=hd)
    want = oracle_mod.attn_decode(q, kb, vb, n_head, n_head_kv, hd, L, threads=8)
    assert_parity(got, want, f"hd={hd} G={n_head // n_head_kv} L={L}")


@pytest.mark.parametrize("n_head,n_head_kv,hd", [(64, 8, 128), (40, 8, 128), (32, 1, 128), (12, 2, 64),
                                                  (10, 2, 256), (56, 8, 64), (14, 2, 128), (48, 8, 128),
                                                  (96, 8, 128), (18, 1, 128)])
def test_decode_large_groups(dev, oracle_mod, n_head, n_head_kv, hd):
    # Groups above 4 (the reference's flash decode limit, src/metal_backend.mm:339): at head_dim
    # 128 groups that are multiples of 4 or 3 run the tuned kernel as units of 4 or 3 heads per
    # KV head (64/8, 96/8, 32/1: units of 4; 48/8, 18/1: units of 3); other groups and head
    # sizes the generic kernel, up to 8 heads per workgroup, larger groups over several.
    L = 1500
    q, kb, vb = _inputs(7 * n_head + hd, n_head, n_head_kv, L, hd=hd)
    got = _run_decode(dev, q, kb, vb, n_head, n_head_kv, L, hd=hd)
    want = oracle_mod.attn_decode(q, kb, vb, n_head, n_head_kv, hd, L, threads=8)
    assert_parity(got, want, f"hd={hd} G={n_head // n_head_kv}")


@pytest.mark.parametrize("hd", [64, 256])
@pytest.mark.parametrize("splits", [1, 2, 5, 32])
def test_decode_split_invariance_head_dims(dev, oracle_mod, hd, splits):
    L = 1200
    q, kb, vb = _inputs(500 + hd, 16, 4, L, hd=hd)
    got = _run_decode(dev, q, kb, vb, 16, 4, L, n_splits=splits, hd=hd)
    want = oracle_mod.attn_decode(q, kb, vb, 16, 4, hd, L)
    assert_parity(got, want, f"hd={hd} splits={splits}")


def test_decode_epochs_across_many_calls(dev, oracle_mod):
    # One workspace, 24 calls whose split counts go up and down: a record slot that an earlier
    # call wrote must never be taken for the current call's (each merger zeroes what it read).
    import ingot_attn as ia

    ws = ia.Workspace(dev)
    rng = np.random.Generator(np.random.PCG64(2024))
    for i in range(24):
        L = int(rng.integers(200, 3000))
        splits = int(rng.choice([0, 2, 7, 16, 31, 32]))
        q, kb, vb = _inputs(900 + i, H, HKV, L)
        got = _run_decode(dev, q, kb, vb, H, HKV, L, n_splits=splits, workspace=ws)
        want = oracle_mod.attn_decode(q, kb, vb, H, HKV, HD, L, threads=8)
        assert_parity(got, want, f"call {i} L={L} splits={splits}")


@pytest.mark.parametrize("n_head,n_head_kv,hd", [(32, 8, 80), (24, 8, 96), (12, 4, 112), (8, 2, 160),
                                                  (4, 4, 20), (2, 1, 1024), (6, 3, 3)])
@pytest.mark.parametrize("L", [1, 300, 2049, 5000])
def test_decode_fallback_head_dims(dev, oracle_mod, n_head, n_head_kv, hd, L):
    # Head sizes without an MFMA kernel run the fallback kernel, the counterpart of the
    # reference's naive attention (shaders/kernels.metal:639-702, src/metal_backend.mm:373-382).
    q, kb, vb = _inputs(60 + L + hd, n_head, n_head_kv, L, n_ctx=L + 3, hd=hd)
    got = _run_decode(dev, q, kb, vb, n_head, n_head_kv, L, hd=hd)
    want = oracle_mod.attn_decode(q, kb, vb, n_head, n_head_kv, hd, L, threads=8)
    assert_parity(got, want, f"fallback hd={hd} G={n_head // n_head_kv} L={L}")
    if L == 1:  # one key: the output is that key's V row, per KV head
        v0 = vb[0].view(np.float16).astype(np.float32).reshape(n_head_kv, hd)
        np.testing.assert_allclose(got.reshape(n_head, hd), np.repeat(v0, n_head // n_head_kv, axis=0), atol=1e-6)


def _counters_all_zero(ws):
    import torch

    torch.cuda.synchronize()
    return int(torch.count_nonzero(ws.buf[:65536]).item()) == 0


def test_decode_handoff_alternating_shapes_one_workspace(dev, oracle_mod):
    # Both decode kernels (tuned: head_dim 128, group <= 4; generic: the rest) on one workspace,
    # head_dims and split counts alternating: records that earlier calls left behind are never
    # taken for the current call's, and every call leaves its completion counters at zero.
    import ingot_attn as ia

    ws = ia.Workspace(dev)
    ws.get(1 << 21)
    shapes = [(24, 8, 128), (32, 8, 64), (16, 8, 256), (64, 8, 128), (12, 2, 64), (24, 8, 128),
              (40, 8, 128), (16, 8, 256), (32, 8, 64)]
    rng = np.random.Generator(np.random.PCG64(77))
    for i in range(27):
        n_head, n_head_kv, hd = shapes[i % len(shapes)]
        L = int(rng.integers(150, 5000))
        splits = int(rng.choice([0, 0, 2, 3, 9, 16, 32]))
        q, kb, vb = _inputs(4000 + i, n_head, n_head_kv, L, hd=hd)
        got = _run_decode(dev, q, kb, vb, n_head, n_head_kv, L, n_splits=splits, hd=hd, workspace=ws)
        want = oracle_mod.attn_decode(q, kb, vb, n_head, n_head_kv, hd, L, threads=8)
        assert_parity(got, want, f"call {i} {n_head}/{n_head_kv} hd={hd} L={L} splits={splits}")
        assert _counters_all_zero(ws), f"call {i}: counters not left at zero"


@pytest.mark.parametrize("n_head,n_head_kv,hd", [(24, 8, 128), (32, 8, 64)])
def test_decode_merge_is_bitwise_reproducible(dev, n_head, n_head_kv, hd):
    # Which key slice merges depends on the order the slices finish in; the merge sums the
    # records in split order whichever it is, so repeated calls are bit-identical.
    import torch
    import ingot_attn as ia

    L = 4096
    q, kb, vb = _inputs(61, n_head, n_head_kv, L, hd=hd)
    qd, kd, vd = _t(q, dev), _t(kb.view(np.int16), dev), _t(vb.view(np.int16), dev)
    desc = ia.decode_desc(n_head, n_head_kv, hd, L)
    outs = []
    for _ in range(16):
        out = torch.empty(n_head * hd, dtype=torch.float32, device=dev)
        ia.attn_decode(qd, kd, vd, out, desc)
        outs.append(out)
    torch.cuda.synchronize()
    ref = outs[0].cpu().numpy().view(np.uint32)
    for o in outs[1:]:
        assert np.array_equal(o.cpu().numpy().view(np.uint32), ref)


def test_decode_closed_forms(dev):
    # single key -> v0; all K equal -> mean of V; dominant key -> its V row
    rng = np.random.Generator(np.random.PCG64(11))
    q = rng.standard_normal(H * HD).astype(np.float32)
    v = rng.standard_normal((300, KV)).astype(np.float16)
    k = np.tile(rng.standard_normal((1, KV)).astype(np.float16), (300, 1))
    got = _run_decode(dev, q, k.view(np.uint16), v.view(np.uint16), H, HKV, 1).reshape(H, HD)
    v0 = v[0].astype(np.float32).reshape(HKV, HD)
    np.testing.assert_allclose(got, np.repeat(v0, 3, axis=0), atol=1e-6)
    got = _run_decode(dev, q, k.view(np.uint16), v.view(np.uint16), H, HKV, 300).reshape(H, HD)
    mean = v.astype(np.float64).reshape(300, HKV, HD).mean(axis=0)
    np.testing.assert_allclose(got, np.repeat(mean, 3, axis=0), atol=1e-5)


def test_decode_and_prefill_share_one_workspace(dev):
    # Decode and split prefill calls keep their records in the same part of one workspace
    # (right after the counters); each call writes the records it reads, so interleaving them
    # changes no bit of any result, and the counters are back at zero after every call.
    import torch
    import ingot_attn as ia

    ws = ia.Workspace(dev)
    ws.get(1 << 24)
    L, pos, n_tok = 3000, 1000, 100
    rng = np.random.Generator(np.random.PCG64(91))
    kb = rng.standard_normal((L, KV)).astype(np.float16).view(np.uint16)
    vb = rng.standard_normal((L, KV)).astype(np.float16).view(np.uint16)
    kd, vd = _t(kb.view(np.int16), dev), _t(vb.view(np.int16), dev)
    qdec = _t(rng.standard_normal(H * HD).astype(np.float32), dev)
    qpre = _t(rng.standard_normal((n_tok, H * HD)).astype(np.float32), dev)
    calls = [("decode", ia.decode_desc(H, HKV, HD, L)),
             ("prefill", ia.prefill_desc(H, HKV, HD, pos, n_tok, n_splits=4)),
             ("decode", ia.decode_desc(H, HKV, HD, 2000, n_splits=7)),
             ("prefill", ia.prefill_desc(H, HKV, HD, pos + 500, n_tok, n_splits=3))]
    assert ia.prefill_splits(calls[1][1]) > 1 and ia.decode_splits(calls[0][1]) > 1

    def run(kind, desc, workspace):
        print(f"[shared-ws] {kind} workspace={'shared' if workspace is ws else 'own'}", flush=True)
        if kind == "decode":
            out = torch.empty(H * HD, dtype=torch.float32, device=dev)
            ia.attn_decode(qdec, kd, vd, out, desc, workspace=workspace)
        else:
            out = torch.empty(n_tok, H * HD, dtype=torch.float32, device=dev)
            ia.attn_prefill(qpre, kd, vd, out, desc, workspace=workspace)
        torch.cuda.synchronize()
        return out.cpu().numpy().view(np.uint32)

    want = [run(k, d, ia.Workspace(dev)) for k, d in calls]
    for rep in range(2):
        for i, (k, d) in enumerate(calls):
            got = run(k, d, ws)
            assert np.array_equal(got, want[i]), f"round {rep}, call {i} ({k}) differs on the shared workspace"
            assert _counters_all_zero(ws), f"round {rep}, call {i} ({k}): counters not left at zero"
