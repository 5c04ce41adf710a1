"""ingot_attn_decode_noalloc (the decode entry point that allocates nothing) against
ingot_attn_decode, through the C ABI: two calls in a row on the library's device-resident
scratch, the second with a smaller input, each bit-identical to the workspace entry point and
within the north-star bar of the CPU oracle; plus its size limit. Collected last (test_zz_*) so
that a failure here cannot hide the other GPU tests."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_parity, ensure_built

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a GPU")
    ensure_built("lib")
    import ingot_attn

    ingot_attn.load_library()
    return torch.device("cuda:0")


def _case(dev, seed, n_head, n_head_kv, hd, L):
    import torch

    rng = np.random.Generator(np.random.PCG64(seed))
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    kb = rng.standard_normal((L, n_head_kv * hd)).astype(np.float16).view(np.uint16)
    vb = rng.standard_normal((L, n_head_kv * hd)).astype(np.float16).view(np.uint16)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return q, kb, vb, t(q), t(kb.view(np.int16)), t(vb.view(np.int16))


@pytest.mark.parametrize("shape", [(24, 8, 128), (32, 8, 64), (16, 8, 256), (64, 8, 128), (24, 8, 96)])
def test_noalloc_matches_workspace_entry_point(dev, oracle_mod, shape):
    import torch
    import ingot_attn as ia

    n_head, n_head_kv, hd = shape
    for i, L in enumerate((4096, 700)):  # the second call is smaller
        print(f"[noalloc] shape={shape} call {i} L={L}", flush=True)
        q, kb, vb, qd, kd, vd = _case(dev, 77 + i, n_head, n_head_kv, hd, L)
        desc = ia.decode_desc(n_head, n_head_kv, hd, L)
        got = torch.full((n_head * hd,), float("nan"), device=dev)
        ia.attn_decode_noalloc(qd, kd, vd, got, desc)
        ref = torch.full_like(got, float("nan"))
        ia.attn_decode(qd, kd, vd, ref, desc, workspace=ia.Workspace(dev))
        torch.cuda.synchronize()
        g, r = got.cpu().numpy(), ref.cpu().numpy()
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), "noalloc differs from ingot_attn_decode"
        want = oracle_mod.attn_decode(q, kb, vb, n_head, n_head_kv, hd, L, threads=8)
        assert_parity(g, want, f"noalloc {shape} L={L}")


def test_noalloc_rejects_more_heads_than_the_scratch_holds(dev):
    import ingot_attn as ia

    lib = ia.load_library()
    big = ia.decode_desc(128, 8, 128, 4096)  # 128 heads, split: more than 64 heads of records
    p = ctypes.c_void_p(1 << 20)
    assert lib.ingot_attn_decode_noalloc(p, p, p, p, ctypes.byref(big), None) == -3
    small_one_split = ia.decode_desc(128, 8, 128, 100)  # one split: counters only, fits
    assert lib.ingot_attn_decode_workspace_size(ctypes.byref(small_one_split)) <= 65536 + 64 * 16896


def test_noalloc_accepts_many_heads_with_one_split(dev, oracle_mod):
    # 128 query heads are more than the scratch's record regions hold, but a one-split call
    # needs no records: the no-allocation entry point takes it and matches ingot_attn_decode.
    import torch
    import ingot_attn as ia

    L = 100
    q, kb, vb, qd, kd, vd = _case(dev, 5, 128, 8, 128, L)
    desc = ia.decode_desc(128, 8, 128, L)
    assert ia.load_library().ingot_attn_decode_splits(ctypes.byref(desc)) == 1
    got = torch.full((128 * 128,), float("nan"), device=dev)
    ia.attn_decode_noalloc(qd, kd, vd, got, desc)
    ref = torch.full_like(got, float("nan"))
    ia.attn_decode(qd, kd, vd, ref, desc, workspace=ia.Workspace(dev))
    torch.cuda.synchronize()
    g, r = got.cpu().numpy(), ref.cpu().numpy()
    assert np.array_equal(g.view(np.uint32), r.view(np.uint32))
    assert_parity(g, oracle_mod.attn_decode(q, kb, vb, 128, 8, 128, L, threads=8), "noalloc 128 heads")
