"""Synthetic Llama-3.2-3B-shaped attention workloads and their seeded inputs.

Shapes (src/model.cpp:38-47 read from GGUF; Llama-3.2-3B, README.md:262): 24 Q heads,
8 KV heads (GQA group 3), head_dim 128, scale 1/sqrt(128). The cache layout is the Metal
backend's: f16 rows [pos][kvh*128 + d] (src/metal_backend.mm:197-198, 437).

Inputs are drawn with numpy's PCG64 generator and `standard_normal` (float64, then cast), so
every consumer that uses the same seed sees bit-identical data. K and V are rounded to f16
with round-to-nearest-even (numpy's float32 -> float16 cast), as `half(x)` does in the
reference's cache writers (shaders/kernels.metal:280-281, 781).
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

N_HEAD = 24
N_HEAD_KV = 8
HEAD_DIM = 128
KV_DIM = N_HEAD_KV * HEAD_DIM
SCALE = 1.0 / math.sqrt(HEAD_DIM)
N_LAYER = 28


@dataclasses.dataclass(frozen=True)
class Workload:
    name: str
    kind: str          # "decode" or "prefill"
    n_keys: int        # cache rows read (decode: pos+1; prefill: pos+n_tok)
    pos: int = 0       # prefill: position of the first query
    n_tok: int = 1     # prefill: queries in the chunk
    kv_scale: float = 1.0
    seed: int = 0

    @property
    def n_ctx(self) -> int:
        return self.n_keys

    def decode_bytes(self) -> int:
        """Algorithmic HBM bytes of one decode call: K+V rows as f16, Q in and O out as f32."""
        return 2 * self.n_keys * KV_DIM * 2 + 2 * N_HEAD * HEAD_DIM * 4

    def pairs(self) -> int:
        """Unmasked (query, key) pairs of a causal prefill chunk: sum_i (pos + i + 1)."""
        n, p = self.n_tok, self.pos
        return n * p + n * (n + 1) // 2

    def prefill_flops(self) -> int:
        """2*hd FLOP for QK^T plus 2*hd for PV per pair and head (softmax excluded)."""
        return 4 * HEAD_DIM * N_HEAD * self.pairs()

    def prefill_bytes(self) -> int:
        """Algorithmic HBM bytes of one prefill call: Q in, O out (f32), K and V rows (f16)."""
        return 2 * self.n_tok * N_HEAD * HEAD_DIM * 4 + 2 * self.n_keys * KV_DIM * 2


# BASELINE.json configs, in order (C1..C5).
C1 = Workload("C1-decode-512", "decode", 512, seed=1)
C2 = Workload("C2-prefill-512@0", "prefill", 512, pos=0, n_tok=512, seed=2)
C3 = Workload("C3-decode-4096", "decode", 4096, kv_scale=0.5, seed=3)
C4 = Workload("C4-prefill-512@3584", "prefill", 4096, pos=3584, n_tok=512, seed=4)
C5_DECODE = tuple(Workload(f"C5-decode-{n}", "decode", n, seed=50 + i)
                  for i, n in enumerate((1024, 2048, 4096, 8192)))
C5_PREFILL = Workload("C5-prefill-2048@6144", "prefill", 8192, pos=6144, n_tok=2048, seed=55)
ALL = (C1, C2, C3, C4) + C5_DECODE + (C5_PREFILL,)
BY_NAME = {w.name: w for w in ALL}


def f16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> IEEE binary16 bit patterns (uint16), round-to-nearest-even."""
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def make_inputs(w: Workload, n_ctx: int | None = None):
    """Returns (q f32 [n_tok][24*128], k_bits u16 [n_ctx][1024], v_bits u16 [n_ctx][1024]).

    Rows n_keys..n_ctx-1 of the cache (if n_ctx > n_keys) are filled with NaN bit patterns:
    they must never be read.
    """
    rng = np.random.Generator(np.random.PCG64(w.seed))
    n_ctx = w.n_keys if n_ctx is None else n_ctx
    n_q = 1 if w.kind == "decode" else w.n_tok
    q = rng.standard_normal((n_q, N_HEAD * HEAD_DIM)).astype(np.float32)
    k = (rng.standard_normal((w.n_keys, KV_DIM)) * w.kv_scale).astype(np.float32)
    v = (rng.standard_normal((w.n_keys, KV_DIM)) * w.kv_scale).astype(np.float32)
    kb = np.full((n_ctx, KV_DIM), 0x7E00, dtype=np.uint16)
    vb = np.full((n_ctx, KV_DIM), 0x7E00, dtype=np.uint16)
    kb[: w.n_keys] = f16_bits(k)
    vb[: w.n_keys] = f16_bits(v)
    return q, kb, vb
