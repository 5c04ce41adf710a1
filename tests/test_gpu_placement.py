"""The memory-order facts the decode split hand-off rests on (inference-agent_amd/csrc/decode_merge.h),
checked on the GPU across XCDs with the probes in inference-agent_amd/probe/bw_probe.hip:

- a relaxed device-scope atomic on one word counts exactly, and returns distinct old values,
  whichever XCD each of thousands of workgroups runs on;
- a device-scope store, a wait for its acknowledgement and a counter increment make the store
  visible to the device-scope loads of the workgroup that counts last, on whichever XCD it runs.

Every kernel here ends on its own; nothing waits for another workgroup."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from conftest import ensure_built

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def probe():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a GPU")
    ensure_built("lib")
    lib = ctypes.CDLL(os.path.join(ROOT, "inference-agent_amd", "libingot_probe.so"))
    for f in (lib.ingot_probe_count, lib.ingot_probe_handoff):
        f.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_uint32, ctypes.c_void_p]
        f.restype = ctypes.c_int
    return lib


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def test_device_scope_atomic_counts_across_xcds(probe):
    import torch

    dev = torch.device("cuda:0")
    n = 4096
    seen_xcds = set()
    for rep in range(4):
        ctr = torch.zeros(64, dtype=torch.int32, device=dev)
        ret = torch.full((n,), -1, dtype=torch.int32, device=dev)
        xcc = torch.full((n,), -1, dtype=torch.int32, device=dev)
        print(f"[placement] count rep {rep} n={n}", flush=True)
        assert probe.ingot_probe_count(_p(ctr), _p(ret), _p(xcc), n, None) == 0
        torch.cuda.synchronize()
        r = ret.cpu().numpy().astype(np.int64)
        assert int(ctr[0].item()) == n
        assert np.array_equal(np.sort(r), np.arange(n))  # every old value exactly once
        seen_xcds |= set(xcc.cpu().numpy().tolist())
    print("XCDs seen:", sorted(seen_xcds))
    assert len(seen_xcds) >= 2  # the counter was shared across XCDs


def test_store_wait_count_load_handoff_across_xcds(probe):
    import torch

    dev = torch.device("cuda:0")
    n = 2048
    mergers = []
    for rep in range(8):
        ctr = torch.zeros(64, dtype=torch.int32, device=dev)
        slot = torch.zeros(n, dtype=torch.int32, device=dev)
        res = torch.zeros(4, dtype=torch.int32, device=dev)
        print(f"[placement] handoff rep {rep} n={n}", flush=True)
        assert probe.ingot_probe_handoff(_p(ctr), _p(slot), _p(res), n, None) == 0
        torch.cuda.synchronize()
        s, bad, x = res.cpu().numpy().astype(np.int64)[:3]
        assert bad == 0 and s == n * (n + 1) // 2, f"rep {rep}: {bad} slots not seen by the last arriver"
        mergers.append(int(x))
    print("last arriver's XCD per run:", mergers)
