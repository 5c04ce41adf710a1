"""The C ABI library: it loads without a GPU, exports every symbol include/*.h declares, its
descriptor structs match the C layout, and its host-side validation behaves as documented.
No compute call is made here (there is no GPU in the CPU suite)."""
from __future__ import annotations

import ctypes
import glob
import os
import re
import subprocess
import tempfile

import pytest

from conftest import PKG, ROOT, ensure_built

INCLUDE = os.path.join(ROOT, "include")


def _declared_functions():
    names = []
    for path in sorted(glob.glob(os.path.join(INCLUDE, "*.h"))):
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(ingot_\w+)\s*\(", text, flags=re.M):
            names.append(m.group(1))
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    ensure_built("lib")
    import ingot_attn

    return ingot_attn.load_library()


def test_header_declares_the_entry_points():
    names = _declared_functions()
    assert "ingot_attn_decode" in names and "ingot_attn_prefill" in names
    import ingot_attn

    assert sorted(ingot_attn.EXPORTS) == sorted(names)


def test_every_declared_symbol_is_exported(lib):
    so = os.path.join(PKG, "libingot_attn.so")
    dyn = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in dyn.splitlines() if line.strip()}
    for name in _declared_functions():
        assert name in exported, f"{name} declared in include/ but not exported"
        assert getattr(lib, name) is not None


def test_struct_layout_matches_c():
    import ingot_attn

    src = r"""
    #include <stdio.h>
    #include <stddef.h>
    #include "ingot_attn.h"
    #include "ingot_linear.h"
    int main(void) {
        printf("%zu %zu %zu %zu %zu\n", sizeof(IngotAttnDecodeDesc),
               offsetof(IngotAttnDecodeDesc, kv_offset), offsetof(IngotAttnDecodeDesc, scale),
               sizeof(IngotAttnPrefillDesc), offsetof(IngotAttnPrefillDesc, kv_offset));
        printf("%zu %zu\n", offsetof(IngotAttnPrefillDesc, q_stride),
               offsetof(IngotAttnPrefillDesc, scale));
        printf("%zu %zu %zu %zu\n", sizeof(IngotRopeKvDesc), offsetof(IngotRopeKvDesc, dst_offset),
               offsetof(IngotRopeKvDesc, q_stride), offsetof(IngotRopeKvDesc, kv_stride));
        printf("%zu %zu %zu\n", sizeof(IngotLinearDesc), offsetof(IngotLinearDesc, accumulate),
               offsetof(IngotLinearDesc, n_splits));
        printf("%zu %zu %zu %zu %zu\n", sizeof(IngotProjDesc), offsetof(IngotProjDesc, n_out),
               offsetof(IngotProjDesc, epilogue), offsetof(IngotProjDesc, eps),
               offsetof(IngotProjDesc, n_tok));
        printf("%d %d %d %d %d\n", INGOT_PROJ_X, INGOT_PROJ_RMSNORM, INGOT_PROJ_STORE,
               INGOT_PROJ_ACCUMULATE, INGOT_PROJ_SILU_GATE);
        return 0;
    }
    """
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "l.c")
        exe = os.path.join(d, "l")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I", INCLUDE, c, "-o", exe], check=True)
        vals = [int(x) for x in subprocess.run([exe], capture_output=True, text=True).stdout.split()]
    D, P, R = ingot_attn.DecodeDesc, ingot_attn.PrefillDesc, ingot_attn.RopeKvDesc
    Li, Pj = ingot_attn.LinearDesc, ingot_attn.ProjDesc
    assert vals == [ctypes.sizeof(D), D.kv_offset.offset, D.scale.offset, ctypes.sizeof(P),
                    P.kv_offset.offset, P.q_stride.offset, P.scale.offset, ctypes.sizeof(R),
                    R.dst_offset.offset, R.q_stride.offset, R.kv_stride.offset, ctypes.sizeof(Li),
                    Li.accumulate.offset, Li.n_splits.offset, ctypes.sizeof(Pj), Pj.n_out.offset,
                    Pj.epilogue.offset, Pj.eps.offset, Pj.n_tok.offset, ingot_attn.PROJ_X, ingot_attn.PROJ_RMSNORM,
                    ingot_attn.PROJ_STORE, ingot_attn.PROJ_ACCUMULATE, ingot_attn.PROJ_SILU_GATE]


def test_host_validation(lib):
    import ingot_attn as ia

    ok = ia.decode_desc(24, 8, 128, 4096)
    assert lib.ingot_attn_decode_workspace_size(ctypes.byref(ok)) > 0
    assert ia.decode_splits(ok) >= 1
    # decode covers every head_dim up to 1024 (64 / 128 / 256 on the MFMA kernels, the others on
    # the fallback kernel, which never splits) and any group size
    for good in (ia.decode_desc(32, 8, 64, 4096), ia.decode_desc(16, 8, 256, 4096),
                 ia.decode_desc(40, 8, 128, 4096), ia.decode_desc(32, 1, 128, 100),
                 ia.decode_desc(24, 8, 96, 4096), ia.decode_desc(4, 2, 1024, 9)):
        assert lib.ingot_attn_decode_workspace_size(ctypes.byref(good)) > 0
    assert ia.decode_splits(ia.decode_desc(24, 8, 96, 4096)) == 16  # key slices of >= 256
    assert ia.decode_splits(ia.decode_desc(24, 8, 96, 1000)) == 4
    assert ia.decode_splits(ia.decode_desc(24, 8, 96, 256)) == 1
    for bad in (ia.decode_desc(24, 8, 1025, 4096), # head_dim above 1024
                ia.decode_desc(24, 7, 128, 4096),  # not divisible
                ia.decode_desc(512, 8, 128, 4096), # more query heads than epoch words
                ia.decode_desc(24, 8, 128, 0)):    # no keys
        assert lib.ingot_attn_decode_workspace_size(ctypes.byref(bad)) == 0
    # null pointers are rejected before any HIP call
    rc = lib.ingot_attn_decode(None, None, None, None, None, 0, ctypes.byref(ok), None)
    assert rc == -1
    rc = lib.ingot_attn_decode(None, None, None, None, None, 0,
                               ctypes.byref(ia.decode_desc(24, 8, 2048, 10)), None)
    assert rc == -2
    # one split needs no records; more splits need a record per (split, head)
    one = ia.decode_desc(24, 8, 128, 100)
    assert lib.ingot_attn_decode_workspace_size(ctypes.byref(one)) == 65536
    s = ia.decode_splits(ok)
    assert s > 1 and lib.ingot_attn_decode_workspace_size(ctypes.byref(ok)) == 65536 + 24 * 32 * (128 * 4 + 16)
    p = ia.prefill_desc(24, 8, 128, 3584, 512)
    assert lib.ingot_attn_prefill_workspace_size(ctypes.byref(p)) > 0
    assert 1 <= ia.prefill_splits(p) <= 16
    bad = ia.prefill_desc(24, 8, 128, 0, 512, q_stride=100)
    assert lib.ingot_attn_prefill_workspace_size(ctypes.byref(bad)) == 0
    assert lib.ingot_attn_strerror(-3).decode().startswith("workspace")
    assert lib.ingot_attn_version().decode().startswith("ingot-attn")


def test_split_resolution(lib):
    import ingot_attn as ia

    for n_keys in (1, 2, 63, 64, 65, 511, 512, 4096, 8192, 100000):
        for req in (0, 1, 3, 64, 5000):
            s = ia.decode_splits(ia.decode_desc(24, 8, 128, n_keys, n_splits=req))
            assert 1 <= s <= min(n_keys, 32)
            s256 = ia.decode_splits(ia.decode_desc(16, 8, 256, n_keys, n_splits=req))
            assert 1 <= s256 <= min(n_keys, 16)
            per = -(-n_keys // s)
            assert (s - 1) * per < n_keys  # no empty split


def test_rope_kv_store_validation(lib):
    """Argument checks of ingot_rope_kv_store run before any HIP call (fake, aligned pointers)."""
    import ingot_attn as ia

    P = ctypes.c_void_p
    a = P(1 << 20)  # 16-byte aligned, never dereferenced: every call below is rejected first
    f = lib.ingot_rope_kv_store
    ok = ia.rope_kv_desc(24, 8, 128, 0, 4)
    assert f(a, None, a, a, a, a, ctypes.byref(ok), None) == -1            # k missing
    assert f(a, a, a, a, a, None, ctypes.byref(ok), None) == -1            # inv_freq missing
    assert f(a, a, a, a, a, a, None, None) == -1                           # no descriptor
    assert f(a, a, a, a, a, a, ctypes.byref(ia.rope_kv_desc(24, 8, 126, 0, 4)), None) == -2
    assert f(a, a, a, a, a, a, ctypes.byref(ia.rope_kv_desc(24, 8, 128, 0, 0)), None) == -1
    assert f(a, a, a, a, a, a, ctypes.byref(ia.rope_kv_desc(24, 8, 128, 0, 4, kv_stride=1000)), None) == -1
    assert f(a, a, a, a, a, a, ctypes.byref(ia.rope_kv_desc(24, 8, 128, 0, 4, q_stride=3000)), None) == -1
    assert f(a, a, a, a, a, a, ctypes.byref(ia.rope_kv_desc(24, 8, 128, 0, 4, dst_offset=2)), None) == -1
    assert f(a, a, P((1 << 20) + 4), a, a, a, ctypes.byref(ok), None) == -1  # misaligned v
    assert f(a, a, a, a, a, a, ctypes.byref(ia.rope_kv_desc(24, 8, 128, 0xffffffff, 2)), None) == -1


def test_linear_descriptor_checks(lib):
    """Weight sizes per GGUF type, split resolution and argument checks of the linear layer
    (no compute call)."""
    import ingot_attn as ia

    n = 3072
    want = {"F32": 4 * n * n, "F16": 2 * n * n, "BF16": 2 * n * n, "Q8_0": n * n // 32 * 34,
            "Q4_0": n * n // 32 * 18, "Q4_1": n * n // 32 * 20, "Q6_K": n * n // 256 * 210}
    for t, nbytes in want.items():
        assert ia.linear_weight_bytes(ia.linear_desc(t, n, n)) == nbytes
    assert ia.linear_weight_bytes(ia.linear_desc(6, 256, 4)) == 0       # Q5_0: no kernel
    assert ia.linear_weight_bytes(ia.linear_desc("Q6_K", 128, 4)) == 0  # n_in % 256
    assert ia.linear_weight_bytes(ia.linear_desc("F16", 48, 4)) == 0    # n_in % 32
    assert ia.linear_weight_bytes(ia.linear_desc("F16", 256, 4, n_splits=9)) == 0
    # one token never splits; small batches split up to 8 ways, never into an empty split,
    # and the workspace covers the chosen split
    assert ia.linear_splits(ia.linear_desc("F16", n, n, 1)) == 1
    for n_tok in (2, 64, 128, 256, 512, 1024, 4096):
        d = ia.linear_desc("Q4_0", n, n, n_tok)
        s = ia.linear_splits(d)
        assert 1 <= s <= 8
        tiles = -(-n // 256) * -(-n_tok // 64)
        assert tiles * s <= max(256, tiles)
        assert ia.linear_workspace_size(d) >= 16384 + (tiles * s * 64 * 256 * 4 if s > 1 else 0)
    assert ia.linear_splits(ia.linear_desc("F16", 256, 256, 64, n_splits=8)) == 1  # 8 k steps min
    assert ia.linear_splits(ia.linear_desc("F16", n, n, 64, n_splits=1)) == 1
    assert ia.linear_splits(ia.linear_desc("F16", n, n, 64, n_splits=3)) == 3
    P = ctypes.c_void_p
    a = P(1 << 20)
    d = ia.linear_desc("F16", 256, 4)
    assert lib.ingot_linear(None, a, a, None, 0, ctypes.byref(d), None) == -1
    assert lib.ingot_linear(P((1 << 20) + 8), a, a, None, 0, ctypes.byref(d), None) == -1  # w align
    assert lib.ingot_linear(a, a, P((1 << 20) + 2), None, 0, ctypes.byref(d), None) == -1  # out align
    assert lib.ingot_linear(a, a, a, None, 0, None, None) == -1


def test_proj_descriptor_checks(lib):
    """Argument checks of the fused one-token projection (no compute call: every case is
    rejected before a launch)."""
    import ingot_attn as ia

    P = ctypes.c_void_p
    a = P(1 << 20)
    arr = lambda *ps: (ctypes.c_void_p * len(ps))(*ps)
    call = lambda d, w=None, x=a, nw=a, out=None: lib.ingot_proj(
        w if w is not None else arr(a, a, a), x, nw, out if out is not None else arr(a, a, a),
        ctypes.byref(d) if d is not None else None, None)
    assert call(None) == -1
    assert call(ia.proj_desc("Q4_0", 3072, [])) == -1                      # no matrix
    bad = ia.proj_desc("Q4_0", 3072, [8, 8, 8]); bad.n_mats = 4
    assert call(bad) == -1                                                 # more than three
    assert call(ia.proj_desc(6, 256, [4])) == -2                           # Q5_0: no kernel
    assert call(ia.proj_desc("Q6_K", 128, [4])) == -2                      # n_in % 256
    assert call(ia.proj_desc("F16", 48, [4])) == -2                        # n_in % 32
    assert call(ia.proj_desc("F16", 256, [4], prologue=2)) == -1
    assert call(ia.proj_desc("F16", 256, [4], epilogue=3)) == -1
    assert call(ia.proj_desc("F16", 256, [4, 0])) == -1                    # empty matrix
    assert call(ia.proj_desc("F16", 256, [4]), x=P((1 << 20) + 4)) == -1   # x align
    assert call(ia.proj_desc("F16", 256, [4]), w=arr(P((1 << 20) + 8))) == -1
    assert call(ia.proj_desc("F16", 256, [4]), out=arr(P((1 << 20) + 2))) == -1
    assert call(ia.proj_desc("F16", 256, [4], prologue=1), nw=None) == -1  # rmsnorm weights
    assert call(ia.proj_desc("F16", 256, [4], prologue=1, eps=-1.0)) == -1
    # the silu gate takes exactly (gate, up) of equal length
    assert call(ia.proj_desc("F16", 256, [4], epilogue=2)) == -1
    assert call(ia.proj_desc("F16", 256, [4, 8], epilogue=2)) == -1
    assert call(ia.proj_desc("F16", 256, [4, 4, 4], epilogue=2)) == -1
    # a chunk takes no rmsnorm prologue (its silu epilogue runs on the GPU: test_gpu_proj.py);
    # a mismatched silu pair is rejected for chunks too
    assert call(ia.proj_desc("F16", 256, [4], prologue=1, eps=1e-5, n_tok=5)) == -2
    assert call(ia.proj_desc("F16", 256, [4, 8], epilogue=2, n_tok=5)) == -1


def test_proj_rope_kv_checks(lib):
    """Argument checks of the fused q/k/v + RoPE + KV-store call (all rejected before a launch)."""
    import ingot_attn as ia

    P = ctypes.c_void_p
    a = P(1 << 20)
    w = (ctypes.c_void_p * 3)(a, a, a)
    good_p = ia.proj_desc("Q4_0", 3072, [3072, 1024, 1024], prologue=ia.PROJ_RMSNORM, eps=1e-5)
    good_r = ia.rope_kv_desc(24, 8, 128, 5, 1, dst_offset=5 * 1024)

    def call(p=good_p, r=good_r, q=a, kc=a, inv=a):
        return lib.ingot_proj_rope_kv(w, a, a, q, a, a, kc, a, inv, ctypes.byref(p) if p is not None else None,
                                      ctypes.byref(r) if r is not None else None, None)

    assert call(p=None) == -1 and call(r=None) == -1
    assert call(p=ia.proj_desc("Q4_0", 3072, [3072, 1024])) == -1             # three matrices
    assert call(p=ia.proj_desc("Q4_0", 3072, [3072, 1024, 1024], epilogue=1)) == -1
    assert call(p=ia.proj_desc("Q4_0", 3072, [3072, 1024, 512])) == -1        # v rows != kv dim
    assert call(r=ia.rope_kv_desc(24, 8, 128, 5, 2)) == -1                      # one token only
    assert call(p=ia.proj_desc("Q4_0", 3072, [3072, 1024, 1024], n_tok=2)) == -1
    assert call(r=ia.rope_kv_desc(24, 8, 130, 5, 1)) in (-1, -2)                # head_dim % 4
    assert call(q=None) == -1 and call(kc=None) == -1 and call(inv=None) == -1
    assert call(q=P((1 << 20) + 4)) == -1                                       # q alignment
    assert call(r=ia.rope_kv_desc(24, 8, 128, 5, 1, dst_offset=2)) == -1      # cache row alignment


def test_prefill_workspace_bound_covers_every_chunk(lib):
    """The prefill split count is not monotonic in the chunk's position (a 317-token chunk at
    2867 needs more records than any chunk at the end of a 4096 context), so the workspace a
    backend allocates once is the documented bound: the longest chunk at the end of the context
    with INGOT_ATTN_MAX_PREFILL_SPLITS splits. Checked here against every chunk length and a
    sweep of positions."""
    import ingot_attn as ia

    text = open(os.path.join(INCLUDE, "ingot_attn.h")).read()
    max_splits = int(re.search(r"#define INGOT_ATTN_MAX_PREFILL_SPLITS (\d+)", text).group(1))

    def size(nh, nkv, hd, pos, n, splits=0):
        d = ia.prefill_desc(nh, nkv, hd, pos, n, n_splits=splits)
        return lib.ingot_attn_prefill_workspace_size(ctypes.byref(d))

    for nh, nkv, hd, n_ctx, n_batch in ((24, 8, 128, 4096, 512), (32, 8, 64, 2048, 256),
                                        (16, 8, 256, 1500, 300), (32, 8, 128, 700, 512)):
        bound = size(nh, nkv, hd, n_ctx - n_batch, n_batch, max_splits)
        for n in range(2, n_batch + 1, 5):
            for pos in range(0, n_ctx - n + 1, 37):
                assert size(nh, nkv, hd, pos, n) <= bound, (nh, nkv, hd, n_ctx, n_batch, pos, n)
