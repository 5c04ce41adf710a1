"""Pins of the CPU linear-layer oracle (oracle/linear_oracle.cpp) without a GPU.

The reference keeps no quantized fixtures (its tests need model files), and src/ops.cpp is
NEON-only, so it cannot be built here. The oracle is pinned instead by:
  - library routines: F16 and BF16 rows against numpy's float16 and a bit shift, Q8_0 against
    d * int8 read with numpy views;
  - round trips: ggml's published quantizers (gguf_blocks.quantize) encode a known matrix; the
    oracle's dequantization must return it within half a quantization step — a swapped nibble,
    a wrong Q6_K element order or scale index gives errors of the order of the values;
  - hand-built blocks with one nonzero element, whose dequantized row has one known entry;
  - the dot products against float64 numpy on the dequantized rows (a dropped block scale or
    a wrong block stride shows up as an O(1) relative error), the accumulate flag, and the f16
    variant against numpy with the two roundings applied by numpy.
"""
from __future__ import annotations

import numpy as np
import pytest

import gguf_blocks as gb

TYPES = ["F32", "F16", "BF16", "Q8_0", "Q4_0", "Q4_1", "Q6_K"]


@pytest.fixture(scope="module")
def orc(oracle_mod):
    return oracle_mod


def _matrix(n_out, n_in, seed=0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n_out, n_in)) * 0.05).astype(np.float32)


def test_float_rows_match_numpy(orc):
    w = _matrix(5, 64)
    got = orc.dequant_rows("F16", gb.quantize("F16", w), 64)
    np.testing.assert_array_equal(got, w.astype(np.float16).astype(np.float32))
    got = orc.dequant_rows("F32", gb.quantize("F32", w), 64)
    np.testing.assert_array_equal(got, w)
    raw = gb.quantize("BF16", w)
    want = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(5, 64)
    np.testing.assert_array_equal(orc.dequant_rows("BF16", raw, 64), want)
    # bf16 keeps 8 significant bits
    assert np.max(np.abs(want - w) / np.abs(w).max()) < 2 ** -7


def test_q8_0_is_scale_times_int8(orc):
    w = _matrix(3, 96, seed=1)
    raw = gb.quantize("Q8_0", w).reshape(3, 3, 34)
    d = raw[..., :2].copy().view(np.float16).astype(np.float32)  # [3, 3, 1]
    q = raw[..., 2:].copy().view(np.int8).astype(np.float32)
    want = (d * q).reshape(3, 96)
    np.testing.assert_array_equal(orc.dequant_rows("Q8_0", raw.reshape(3, -1), 96), want)


@pytest.mark.parametrize("t", ["Q8_0", "Q4_0", "Q4_1", "Q6_K"])
def test_round_trip_within_half_a_step(orc, t):
    n_in = 512
    w = _matrix(7, n_in, seed=2)
    got = orc.dequant_rows(t, gb.quantize(t, w), n_in)
    err = np.abs(got - w)
    if t in ("Q8_0", "Q4_0", "Q4_1"):
        blocks = w.reshape(7, -1, 32)
        if t == "Q8_0":
            step = np.abs(blocks).max(axis=2) / 127
        elif t == "Q4_0":
            # d = max/-8 maps the largest-magnitude value to -8; values of the other sign near
            # that magnitude clip at +7, a full step away (ggml's quantize_row_q4_0)
            step = np.abs(blocks).max(axis=2) / 8 * 2
        else:
            step = (blocks.max(axis=2) - blocks.min(axis=2)) / 15
        bound = np.repeat(step * 0.5, 32, axis=1) * 1.01 + 1e-3 * np.abs(w) + 1e-7
    else:
        sub = np.abs(w.reshape(7, -1, 16)).max(axis=2) / 31  # ~ the step of each 16 elements
        bound = np.repeat(sub * 0.5 + np.abs(sub).max() / 127 * 16, 16, axis=1) + 1e-7
    assert np.all(err <= bound), f"{t}: max err {err.max():.3e}"
    # and the encoding is far from trivial: a shuffled order would not pass
    assert np.abs(got - np.roll(w, 1, axis=1)).max() > 10 * err.max()


def test_q4_0_single_nibbles(orc):
    # d = 1.0; byte j = 0x88 except one: element 3 -> low nibble of byte 3, element 19 -> its
    # high nibble. nibble 8 decodes to 0.
    blk = np.zeros(18, dtype=np.uint8)
    blk[0:2] = np.array([1.0], dtype=np.float16).view(np.uint8)
    blk[2:] = 0x88
    blk[2 + 3] = 0x8B          # element 3 = 11 - 8 = 3
    got = orc.dequant_rows("Q4_0", blk[None], 32)[0]
    want = np.zeros(32, np.float32)
    want[3] = 3
    np.testing.assert_array_equal(got, want)
    blk[2 + 3] = 0x28          # element 19 = 2 - 8 = -6
    got = orc.dequant_rows("Q4_0", blk[None], 32)[0]
    want[:] = 0
    want[19] = -6
    np.testing.assert_array_equal(got, want)


def test_q6_k_single_element(orc):
    # Element 32*2 + 5 of the second half (e = 128 + 69 = 197): g = 2 -> high nibble of
    # ql[64 + 5], bits 4-5 of qh[32 + 5], scale index 8 + 0 + 4 = 12 (e // 16 = 12).
    blk = np.zeros(210, dtype=np.uint8)
    for i in range(128):
        blk[i] = 0x00
    # every element's q6 = 32 (decodes to 0): low 4 bits 0, high 2 bits 2 -> qh = 0b10101010
    blk[128:192] = 0xAA
    blk[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)
    blk[208:210] = np.array([0.5], dtype=np.float16).view(np.uint8)
    # element 197: q6 = 32 + 7 = 39 = 0b100111 -> low nibble 7 (high nibble of ql[69]), high bits 2
    blk[64 + 5] = 0x70
    got = orc.dequant_rows("Q6_K", blk[None], 256)[0]
    want = np.zeros(256, np.float32)
    want[197] = 0.5 * 13 * 7
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("t", TYPES)
def test_linear_matches_float64(orc, t):
    n_in, n_out, n_tok = 512, 48, 3
    raw = gb.random_weights(t, n_out, n_in, seed=3)
    x = np.random.default_rng(4).standard_normal((n_tok, n_in)).astype(np.float32)
    deq = orc.dequant_rows(t, raw, n_in).astype(np.float64)
    want = x.astype(np.float64) @ deq.T
    got = orc.linear(t, raw, x, n_in, n_out)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.abs(want).max() + 1e-6
    # accumulate adds onto the existing contents (the residual add after wo)
    base = np.random.default_rng(5).standard_normal((n_tok, n_out)).astype(np.float32)
    acc = orc.linear(t, raw, x, n_in, n_out, out=base, accumulate=True)
    np.testing.assert_allclose(acc, base + got, rtol=0, atol=1e-6)


@pytest.mark.parametrize("t", TYPES)
def test_f16_path_matches_numpy(orc, t):
    n_in, n_out, n_tok = 256, 16, 4
    raw = gb.random_weights(t, n_out, n_in, seed=6)
    x = np.random.default_rng(7).standard_normal((n_tok, n_in)).astype(np.float32)
    deq = orc.dequant_rows(t, raw, n_in)
    wh = deq.astype(np.float16).astype(np.float64)
    xh = x.astype(np.float16).astype(np.float64)
    want = xh @ wh.T
    got = orc.linear(t, raw, x, n_in, n_out, f16_path=True)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.abs(want).max()
    # and it differs from the f32 path by about the f16 rounding only
    f32 = orc.linear(t, raw, x, n_in, n_out)
    rel = np.linalg.norm(got - f32) / np.linalg.norm(f32)
    assert rel < 2e-3


def test_bad_arguments(orc):
    with pytest.raises(ValueError):
        orc.dequant_rows("Q4_0", np.zeros(18, np.uint8), 16)  # n not a block multiple
    with pytest.raises(KeyError):
        orc.dequant_rows("Q5_0", np.zeros(22, np.uint8), 32)
