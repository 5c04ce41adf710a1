"""The committed fixtures (tests/golden/) against the oracle (CPU) and the HIP library (GPU)."""
import hashlib
import os

import numpy as np
import pytest

from conftest import ROOT, assert_parity, ensure_built

GOLD = os.path.join(ROOT, "tests", "golden")
SMALL = ["small_decode_g3.npz", "small_prefill_g3.npz", "small_prefill_g2.npz"]


@pytest.mark.parametrize("name", SMALL)
def test_oracle_reproduces_small_fixtures(oracle_mod, name):
    f = np.load(os.path.join(GOLD, name))
    out = oracle_mod.attn_prefill(f["q"], f["k"], f["v"], int(f["n_head"]), int(f["n_head_kv"]), 128,
                                  int(f["pos"]), int(f["n_tok"]))
    assert np.array_equal(out, f["out"])


@pytest.mark.parametrize("wname", ["C1-decode-512", "C3-decode-4096"])
def test_seeded_inputs_and_oracle_output_are_stable(oracle_mod, wname):
    import workloads as W

    w = W.BY_NAME[wname]
    f = np.load(os.path.join(GOLD, f"{wname}.npz"))
    q, kb, vb = W.make_inputs(w)
    assert hashlib.sha256(q.tobytes() + kb.tobytes() + vb.tobytes()).hexdigest() == str(f["digest"])
    out = oracle_mod.attn_decode(q, kb, vb, 24, 8, 128, w.n_keys, threads=4)
    assert np.array_equal(out, f["out"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", SMALL)
def test_gpu_matches_small_fixtures(name):
    import torch

    ensure_built("lib")
    import ingot_attn as ia

    f = np.load(os.path.join(GOLD, name))
    dev = torch.device("cuda:0")
    H, HKV, pos, n = int(f["n_head"]), int(f["n_head_kv"]), int(f["pos"]), int(f["n_tok"])
    print(f"[golden] {name} H={H} HKV={HKV} pos={pos} n_tok={n}", flush=True)
    q = torch.from_numpy(f["q"]).to(dev)
    k = torch.from_numpy(f["k"].view(np.int16)).to(dev)
    v = torch.from_numpy(f["v"].view(np.int16)).to(dev)
    out = torch.full_like(q, float("nan"))
    if n == 1:
        ia.attn_decode(q[0], k, v, out[0], ia.decode_desc(H, HKV, 128, pos + 1))
    else:
        ia.attn_prefill(q, k, v, out, ia.prefill_desc(H, HKV, 128, pos, n))
    torch.cuda.synchronize()
    assert_parity(out.cpu().numpy(), f["out"], name)


@pytest.mark.gpu
@pytest.mark.parametrize("wname", ["C1-decode-512", "C3-decode-4096"])
def test_gpu_matches_config_fixtures(wname):
    import torch

    ensure_built("lib")
    import ingot_attn as ia
    import workloads as W

    w = W.BY_NAME[wname]
    f = np.load(os.path.join(GOLD, f"{wname}.npz"))
    q, kb, vb = W.make_inputs(w)
    dev = torch.device("cuda:0")
    print(f"[golden] {wname}", flush=True)
    out = torch.empty(24 * 128, dtype=torch.float32, device=dev)
    ia.attn_decode(torch.from_numpy(q[0]).to(dev), torch.from_numpy(kb.view(np.int16)).to(dev),
                   torch.from_numpy(vb.view(np.int16)).to(dev), out, ia.decode_desc(24, 8, 128, w.n_keys))
    torch.cuda.synchronize()
    assert_parity(out.cpu().numpy(), f["out"], wname)
