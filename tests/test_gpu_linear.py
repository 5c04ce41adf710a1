"""GPU parity of the linear layer (ingot_linear) against the CPU oracle, every weight type.

Tolerances, stated per path:
  - one token (matvec, f32 arithmetic on exactly dequantized weights): against oracle_linear
    (ops::matvec), rel-L2 <= 1e-5 and max|d| <= 1e-5 * max|ref| + 1e-6 — only the order of the
    f32 sums differs;
  - several tokens (MFMA matmul, x and weights rounded to f16 as the reference's Metal batched
    path does): against oracle_linear_f16 (the same two roundings on the CPU), rel-L2 <= 1e-5 and
    max|d| <= 1e-5 * max|ref| + 1e-6; against the f32 CPU path
    max|d| <= 2e-3 and rel-L2 <= 1e-3 (outputs are O(1): x ~ N(0,1), W rows of norm ~1);
  - out_offset and accumulate: out = base + W·x in the addressed range, every element outside
    it keeps its NaN canary bits.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_parity, ensure_built

import gguf_blocks as gb

pytestmark = pytest.mark.gpu

TYPES = ["F32", "F16", "BF16", "Q8_0", "Q4_0", "Q4_1", "Q6_K"]


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


def _run(dev, t, raw, x, n_in, n_out, base=None, out_offset=0, pad=37, use_workspace=True):
    """Runs ingot_linear; returns (result [n_tok][n_out], the whole out buffer)."""
    import torch
    import ingot_attn as ia

    n_tok = x.shape[0]
    total = out_offset + n_tok * n_out + pad
    buf = np.full(total, np.nan, dtype=np.float32)
    if base is not None:
        buf[out_offset:out_offset + n_tok * n_out] = base.ravel()
    out = _t(buf, dev)
    d = ia.linear_desc(t, n_in, n_out, n_tok, out_offset=out_offset, accumulate=base is not None)
    assert ia.linear_weight_bytes(d) == raw.size
    ia.linear(_t(raw.reshape(-1), dev), _t(x, dev), out, d, use_workspace=use_workspace)
    torch.cuda.synchronize()
    full = out.cpu().numpy()
    return full[out_offset:out_offset + n_tok * n_out].reshape(n_tok, n_out), full


def _close(got, want, what):
    d = np.abs(got.astype(np.float64) - want)
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    tol = 1e-5 * np.abs(want).max() + 1e-6
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert d.max() <= tol and rel <= 1e-5, f"{what}: max|d|={d.max():.3e} (tol {tol:.1e}), rel-L2={rel:.3e}"


def _x(n_tok, n_in, seed):
    return np.random.default_rng(seed).standard_normal((n_tok, n_in)).astype(np.float32)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_in,n_out", [(3072, 3072), (256, 200), (8192, 96), (512, 1001), (256, 1001),
                                         (768, 3)])
def test_matvec(dev, oracle_mod, t, n_in, n_out):
    raw = gb.random_weights(t, n_out, n_in, seed=n_in + n_out)
    x = _x(1, n_in, seed=1)
    got, _ = _run(dev, t, raw, x, n_in, n_out)
    _close(got, oracle_mod.linear(t, raw, x, n_in, n_out), f"{t} matvec {n_in}x{n_out}")


@pytest.mark.parametrize("t", TYPES)
def test_matvec_long_rows(dev, oracle_mod, t):
    """A 28672-wide row (a 70B-class down projection): x alone takes 112 KB of the staging LDS,
    so the staged kernel falls back to one row per workgroup."""
    n_in, n_out = 28672, 67
    raw = gb.random_weights(t, n_out, n_in, seed=5)
    x = _x(1, n_in, seed=6)
    got, _ = _run(dev, t, raw, x, n_in, n_out)
    _close(got, oracle_mod.linear(t, raw, x, n_in, n_out), f"{t} matvec {n_in}x{n_out}")


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_tok,n_in,n_out", [(2, 256, 256), (37, 512, 300), (64, 1024, 512),
                                              (130, 768, 257)])
def test_matmul(dev, oracle_mod, t, n_tok, n_in, n_out):
    raw = gb.random_weights(t, n_out, n_in, seed=n_tok + n_in)
    x = _x(n_tok, n_in, seed=2)
    got, _ = _run(dev, t, raw, x, n_in, n_out)
    _close(got, oracle_mod.linear(t, raw, x, n_in, n_out, f16_path=True),
           f"{t} matmul {n_tok}x{n_in}x{n_out}")
    assert_parity(got, oracle_mod.linear(t, raw, x, n_in, n_out), f"{t} matmul vs f32 path")


@pytest.mark.parametrize("t", ["F16", "Q4_0", "Q8_0", "Q6_K"])
def test_wo_prefill_shape(dev, oracle_mod, t):
    """The attention output projection at the 512-token prefill chunk, with the residual add."""
    n_tok, n = 512, 3072
    raw = gb.random_weights(t, n, n, seed=11)
    x = _x(n_tok, n, seed=12)
    base = _x(n_tok, n, seed=13)
    got, _ = _run(dev, t, raw, x, n, n, base=base)
    want = oracle_mod.linear(t, raw, x, n, n, out=base, accumulate=True, f16_path=True)
    _close(got, want, f"{t} wo 512x3072x3072")


@pytest.mark.parametrize("n_tok", [1, 5])
def test_offset_and_accumulate(dev, oracle_mod, n_tok):
    t, n_in, n_out, off = "Q4_0", 512, 96, 1234
    raw = gb.random_weights(t, n_out, n_in, seed=21)
    x = _x(n_tok, n_in, seed=22)
    base = _x(n_tok, n_out, seed=23)
    got, full = _run(dev, t, raw, x, n_in, n_out, base=base, out_offset=off)
    want = oracle_mod.linear(t, raw, x, n_in, n_out, out=base, accumulate=True, f16_path=n_tok > 1)
    _close(got, want, f"accumulate n_tok={n_tok}")
    assert np.all(np.isnan(full[:off])) and np.all(np.isnan(full[off + n_tok * n_out:]))
    # without accumulate the previous contents are ignored
    got2, _ = _run(dev, t, raw, x, n_in, n_out, out_offset=off)
    _close(got2, oracle_mod.linear(t, raw, x, n_in, n_out, f16_path=n_tok > 1), "overwrite")


def test_errors(dev):
    import torch
    import ingot_attn as ia

    lib = ia.load_library()
    w = torch.zeros(4096, dtype=torch.uint8, device=dev)
    x = torch.zeros(256, dtype=torch.float32, device=dev)
    o = torch.zeros(256, dtype=torch.float32, device=dev)
    import ctypes

    def call(d, ws=None):
        return lib.ingot_linear(ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                ctypes.c_void_p(o.data_ptr()), ws, 0, ctypes.byref(d), None)

    assert call(ia.linear_desc(6, 256, 4)) == -2          # Q5_0: no kernel
    assert call(ia.linear_desc("Q6_K", 128, 4)) == -2     # n_in not a multiple of 256
    assert call(ia.linear_desc("F16", 0, 4)) == -1
    assert call(ia.linear_desc("F16", 256, 4)) == 0
    assert call(ia.linear_desc("F16", 256, 4), ws=ctypes.c_void_p(o.data_ptr() + 4)) == -1  # misaligned
    torch.cuda.synchronize()


@pytest.mark.parametrize("n_tok", [2, 64, 128, 512])
def test_split_k_is_deterministic(dev, oracle_mod, n_tok):
    """Small batches split n_in across workgroups (up to 8 ways); the result is the same on
    every call (fixed-order partial sums, counters left at zero) and within f32 rounding of
    the unsplit call; both match the f16-path oracle."""
    import ingot_attn as ia

    t, n = "Q4_0", 3072
    d = ia.linear_desc(t, n, n, n_tok)
    assert ia.linear_workspace_size(d) >= 16384
    raw = gb.random_weights(t, n, n, seed=31)
    x = _x(n_tok, n, seed=32)
    a, _ = _run(dev, t, raw, x, n, n)
    b, _ = _run(dev, t, raw, x, n, n)
    c, _ = _run(dev, t, raw, x, n, n, use_workspace=False)
    assert ia.linear_splits(d) > 1 or n_tok >= 512
    np.testing.assert_array_equal(a, b)
    _close(a, c, f"split vs unsplit n_tok={n_tok}")
    _close(a, oracle_mod.linear(t, raw, x, n, n, f16_path=True), f"split n_tok={n_tok}")


@pytest.mark.parametrize("t", ["Q8_0", "Q6_K"])
@pytest.mark.parametrize("n_splits", [2, 3, 5, 8])
def test_requested_splits(dev, oracle_mod, t, n_splits):
    """An explicit split count (uneven last split for 3 and 5 over 96 k steps) gives the same
    result as no split, within f32 rounding, and matches the oracle. (Q6_K: a split starts at a
    210-byte block boundary, so each split's LDS windows sit at their own shifts.)"""
    import torch
    import ingot_attn as ia

    n, n_tok = 3072, 100
    raw = gb.random_weights(t, n, n, seed=41)
    x = _x(n_tok, n, seed=42)
    d = ia.linear_desc(t, n, n, n_tok, n_splits=n_splits)
    assert ia.linear_splits(d) == n_splits
    out = _t(np.zeros((n_tok, n), np.float32), dev)
    ia.linear(_t(raw.reshape(-1), dev), _t(x, dev), out, d)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref, _ = _run(dev, t, raw, x, n, n, use_workspace=False)
    _close(got, ref, f"n_splits={n_splits} vs unsplit")
    _close(got, oracle_mod.linear(t, raw, x, n, n, f16_path=True), f"n_splits={n_splits}")


@pytest.mark.parametrize("t", ["F16", "BF16", "F32", "Q4_0", "Q4_1", "Q6_K"])
@pytest.mark.parametrize("n_out", [2000, 2001])
def test_batched_128_token_tiles(dev, oracle_mod, t, n_out):
    """Enough token tiles for two rounds of 64-token tiles take one round of 128-token tiles
    (waves of 64 tokens x 64 rows); ragged n_tok and n_out (2001: rows not 16-byte aligned, the
    scalar output path), with the residual add. Matches the f16-path oracle. (Q6_K rows of 210
    bytes: the last tile's last block ends inside a 16-byte chunk.)"""
    n_in, n_tok = 256, 2100  # 8 x 33 tiles of 64 tokens, 8 x 17 of 128
    raw = gb.random_weights(t, n_out, n_in, seed=55)
    x = _x(n_tok, n_in, seed=56)
    base = np.random.default_rng(57).standard_normal(n_tok * n_out).astype(np.float32)
    got, _ = _run(dev, t, raw, x, n_in, n_out, base=base)
    want = oracle_mod.linear(t, raw, x, n_in, n_out, f16_path=True) + base.reshape(n_tok, n_out)
    _close(got, want, f"{t} 128-token tiles")
