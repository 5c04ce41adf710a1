"""Synthetic GGUF weight matrices: f32 values encoded in the on-disk block layouts.

Test and bench data only (there are no model files on the GPU box). The layouts are the ones
the reference reads (src/ops.cpp:33-87, shaders/kernels.metal:11-17); the quantizers follow
ggml's published reference quantizers (quantize_row_q8_0 / q4_0 / q4_1 in ggml-quants.c), and
Q6_K uses a plain per-16-element max-abs scale with an int8 super-scale (a valid Q6_K encoding,
not ggml's iterative search). All return a uint8 array [n_out][row_bytes].
"""
from __future__ import annotations

import numpy as np

TYPES = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q8_0": 8, "Q6_K": 14, "BF16": 30}
BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 8: (32, 34), 2: (32, 18), 3: (32, 20), 14: (256, 210)}


def type_id(t) -> int:
    return TYPES[t] if isinstance(t, str) else int(t)


def row_bytes(t, n_in: int) -> int:
    be, bb = BLOCK[type_id(t)]
    return n_in // be * bb


def _f16(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).astype(np.float16)


def _round_away(a: np.ndarray) -> np.ndarray:
    """C roundf: halves away from zero."""
    return np.sign(a) * np.floor(np.abs(a) + 0.5)


def quantize(t, w: np.ndarray) -> np.ndarray:
    """Encodes w ([n_out][n_in] f32) in type t; returns the bytes [n_out][row_bytes]."""
    t = type_id(t)
    w = np.ascontiguousarray(w, dtype=np.float32)
    n_out, n_in = w.shape
    be, bb = BLOCK[t]
    assert n_in % be == 0
    if t == 0:
        return w.view(np.uint8).reshape(n_out, -1).copy()
    if t == 1:
        return _f16(w).view(np.uint8).reshape(n_out, -1).copy()
    if t == 30:  # bf16: round to nearest even on the top 16 bits
        u = w.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        return r.view(np.uint8).reshape(n_out, -1).copy()
    blocks = w.reshape(n_out, n_in // be, be)
    nb = blocks.shape[1]
    out = np.zeros((n_out, nb, bb), dtype=np.uint8)
    if t == 8:
        amax = np.abs(blocks).max(axis=2)
        d = amax / 127.0
        inv = np.where(d != 0, 1.0 / np.where(d != 0, d, 1), 0.0)
        q = _round_away(blocks * inv[..., None]).astype(np.int8)
        out[..., 0:2] = _f16(d).view(np.uint8).reshape(n_out, nb, 2)
        out[..., 2:34] = q.view(np.uint8)
    elif t == 2:
        idx = np.abs(blocks).argmax(axis=2)
        mx = np.take_along_axis(blocks, idx[..., None], axis=2)[..., 0]
        d = mx / -8.0
        inv = np.where(d != 0, 1.0 / np.where(d != 0, d, 1), 0.0)
        q = np.minimum(15, np.trunc(blocks * inv[..., None] + 8.5)).astype(np.uint8)
        out[..., 0:2] = _f16(d).view(np.uint8).reshape(n_out, nb, 2)
        out[..., 2:18] = q[..., :16] | (q[..., 16:] << 4)
    elif t == 3:
        mn = blocks.min(axis=2)
        mx = blocks.max(axis=2)
        d = (mx - mn) / 15.0
        inv = np.where(d != 0, 1.0 / np.where(d != 0, d, 1), 0.0)
        q = np.minimum(15, np.trunc((blocks - mn[..., None]) * inv[..., None] + 0.5)).astype(np.uint8)
        out[..., 0:2] = _f16(d).view(np.uint8).reshape(n_out, nb, 2)
        out[..., 2:4] = _f16(mn).view(np.uint8).reshape(n_out, nb, 2)
        out[..., 4:20] = q[..., :16] | (q[..., 16:] << 4)
    elif t == 14:
        sub = blocks.reshape(n_out, nb, 16, 16)
        scale = np.abs(sub).max(axis=3) / 31.0                      # per 16 elements
        dsup = np.abs(scale).max(axis=2) / 127.0                   # per block
        d16 = _f16(dsup).astype(np.float32)
        sc = np.where(d16[..., None] != 0, _round_away(scale / np.where(d16 != 0, d16, 1)[..., None]), 0)
        sc = np.clip(sc, -128, 127).astype(np.int8)
        step = d16[..., None] * sc.astype(np.float32)
        q = np.where(step[..., None] != 0, _round_away(sub / np.where(step != 0, step, 1)[..., None]), 0)
        q = (np.clip(q, -32, 31) + 32).astype(np.uint8).reshape(n_out, nb, 256)
        e = np.arange(256)
        h, r = e // 128, e % 128
        g, l = r // 32, r % 32
        ql_idx = h * 64 + l + 32 * (g & 1)
        qh_idx = h * 32 + l
        ql = np.zeros((n_out, nb, 128), dtype=np.uint8)
        qh = np.zeros((n_out, nb, 64), dtype=np.uint8)
        lo = q & 0xF
        hi = q >> 4
        for i in range(256):
            ql[..., ql_idx[i]] |= (lo[..., i] << np.uint8(0 if g[i] < 2 else 4)).astype(np.uint8)
            qh[..., qh_idx[i]] |= (hi[..., i] << np.uint8(2 * g[i])).astype(np.uint8)
        out[..., 0:128] = ql
        out[..., 128:192] = qh
        out[..., 192:208] = sc.view(np.uint8)
        out[..., 208:210] = _f16(dsup).view(np.uint8).reshape(n_out, nb, 2)
    return out.reshape(n_out, nb * bb)


def random_weights(t, n_out: int, n_in: int, seed: int = 0, scale: float | None = None) -> np.ndarray:
    """N(0, scale^2) weights (default scale 1/sqrt(n_in)) encoded in type t."""
    rng = np.random.default_rng(seed)
    s = 1.0 / np.sqrt(n_in) if scale is None else scale
    return quantize(t, (rng.standard_normal((n_out, n_in)) * s).astype(np.float32))
