"""Runs the plain copy probe (libingot_probe.so, probe_copy) over a buffer of known size, to
calibrate rocprofv3's FETCH_SIZE / WRITE_SIZE counters against bytes actually moved:
    rocprofv3 --pmc FETCH_SIZE -- python3 inference-agent_amd/probe/copy_probe.py [MiB]
Each dispatch copies exactly MiB mebibytes (reads MiB, writes MiB)."""
import ctypes
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
lib = ctypes.CDLL(os.path.join(HERE, "..", "libingot_probe.so"))
lib.ingot_probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_void_p]
mib = int(sys.argv[1]) if len(sys.argv) > 1 else 64
n = mib << 20
src = torch.ones(n // 4, device="cuda")
dst = torch.empty_like(src)
for _ in range(5):
    rc = lib.ingot_probe_copy(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), n, 2048,
                              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
torch.cuda.synchronize()
assert bool((dst == 1).all())
print(f"copied {mib} MiB x 5")
