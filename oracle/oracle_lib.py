"""ctypes binding of liboracle.so — the CPU restatement of Ingot's attention.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker and the CPU baseline. The product path never imports it.
Reference lines each function follows are cited in attn_oracle.cpp.
"""
from __future__ import annotations

import ctypes
import math
import os
from ctypes import c_float, c_int, c_size_t, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_f32_to_f16.argtypes = [c_void_p, c_void_p, c_size_t]
        L.oracle_f16_to_f32.argtypes = [c_void_p, c_void_p, c_size_t]
        L.oracle_softmax.argtypes = [c_void_p, c_size_t]
        L.oracle_attn_decode.argtypes = [c_void_p] * 4 + [c_int] * 4 + [c_float, c_int]
        L.oracle_attn_decode.restype = c_int
        L.oracle_attn_prefill.argtypes = [c_void_p] * 4 + [c_int] * 6 + [c_float, c_int]
        L.oracle_attn_prefill.restype = c_int
        L.oracle_rope_inv_freq.argtypes = [c_float, c_int, c_void_p, c_void_p]
        L.oracle_rope.argtypes = [c_void_p] + [c_int] * 5 + [c_void_p]
        L.oracle_rope_kv_store.argtypes = ([c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p,
                                            c_void_p, c_size_t] + [c_int] * 4 + [c_void_p])
        L.oracle_rope_kv_store.restype = c_int
        L.oracle_rmsnorm.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_int, c_float]
        L.oracle_silu_mul.argtypes = [c_void_p, c_void_p, c_size_t]
        L.oracle_dequant_row.argtypes = [c_int, c_void_p, c_void_p, c_int]
        L.oracle_dequant_row.restype = c_int
        for f in (L.oracle_linear, L.oracle_linear_f16):
            f.argtypes = [c_int, c_void_p, c_void_p, c_void_p] + [c_int] * 5
            f.restype = c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return c_void_p(a.ctypes.data)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16(_ptr(x), _ptr(out), x.size)
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oracle_f16_to_f32(_ptr(h), _ptr(out), h.size)
    return out


def softmax(x: np.ndarray) -> np.ndarray:
    x = np.array(x, dtype=np.float32, copy=True)
    lib().oracle_softmax(_ptr(x), x.size)
    return x


def attn_decode(q, k_bits, v_bits, n_head, n_head_kv, head_dim, n_keys, scale=None, threads=1):
    """q f32 [n_head*hd]; k_bits/v_bits u16 [>= n_keys][n_head_kv*hd] -> out f32 [n_head*hd]."""
    scale = 1.0 / math.sqrt(head_dim) if scale is None else scale
    q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
    k_bits = np.ascontiguousarray(k_bits, dtype=np.uint16)
    v_bits = np.ascontiguousarray(v_bits, dtype=np.uint16)
    out = np.empty(n_head * head_dim, dtype=np.float32)
    rc = lib().oracle_attn_decode(_ptr(q), _ptr(k_bits), _ptr(v_bits), _ptr(out), n_head,
                                  n_head_kv, head_dim, n_keys, scale, threads)
    if rc != 0:
        raise ValueError("oracle_attn_decode: bad arguments")
    return out


def attn_prefill(q, k_bits, v_bits, n_head, n_head_kv, head_dim, pos, n_tok, scale=None,
                 threads=1):
    """q f32 [n_tok][n_head*hd]; cache rows 0..pos+n_tok-1 -> out f32 [n_tok][n_head*hd]."""
    scale = 1.0 / math.sqrt(head_dim) if scale is None else scale
    q = np.ascontiguousarray(q, dtype=np.float32).reshape(n_tok, -1)
    k_bits = np.ascontiguousarray(k_bits, dtype=np.uint16)
    v_bits = np.ascontiguousarray(v_bits, dtype=np.uint16)
    out = np.zeros_like(q)
    rc = lib().oracle_attn_prefill(_ptr(q), _ptr(k_bits), _ptr(v_bits), _ptr(out), n_head,
                                   n_head_kv, head_dim, pos, n_tok, q.shape[1], scale, threads)
    if rc != 0:
        raise ValueError("oracle_attn_prefill: bad arguments")
    return out


def rope_inv_freq(theta: float, head_dim: int, factors=None) -> np.ndarray:
    """src/model.cpp:59-68: head_dim/2 rotary frequencies."""
    out = np.empty(head_dim // 2, dtype=np.float32)
    f = None if factors is None else np.ascontiguousarray(factors, dtype=np.float32)
    lib().oracle_rope_inv_freq(theta, head_dim, None if f is None else _ptr(f), _ptr(out))
    return out


def rope(x, n_heads, head_dim, pos, inv_freq) -> np.ndarray:
    """ops::rope (src/ops.cpp:243-255) on rows x [n_tok][row_stride], token t at pos + t."""
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    x2 = x.reshape(x.shape[0], -1) if x.ndim > 1 else x.reshape(1, -1)
    inv_freq = np.ascontiguousarray(inv_freq, dtype=np.float32)
    lib().oracle_rope(_ptr(x2), x2.shape[0], x2.shape[1], n_heads, head_dim, pos, _ptr(inv_freq))
    return x


def rope_kv_store(q, k, v, k_cache, v_cache, dst_offset, n_head, n_head_kv, head_dim, pos,
                  inv_freq):
    """RoPE on q (returned, or None) and k; K, V as f16 into copies of the caches (returned)."""
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    n_tok = k.shape[0]
    kc = np.array(k_cache, dtype=np.uint16, copy=True, order="C")
    vc = np.array(v_cache, dtype=np.uint16, copy=True, order="C")
    qq = None if q is None else np.array(q, dtype=np.float32, copy=True, order="C")
    inv_freq = np.ascontiguousarray(inv_freq, dtype=np.float32)
    rc = lib().oracle_rope_kv_store(None if qq is None else _ptr(qq), 0 if qq is None else qq.shape[1],
                                    n_head, _ptr(k), _ptr(v), k.shape[1], _ptr(kc), _ptr(vc),
                                    dst_offset, n_head_kv, head_dim, pos, n_tok, _ptr(inv_freq))
    if rc != 0:
        raise ValueError("oracle_rope_kv_store: bad arguments")
    return qq, kc, vc


# GGUF type ids and (elements, bytes) per block, as in the library (src/gguf.h:30-33).
GGUF_TYPES = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q8_0": 8, "Q6_K": 14, "BF16": 30}
BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 8: (32, 34), 2: (32, 18), 3: (32, 20), 14: (256, 210)}


def _type_id(t):
    return GGUF_TYPES[t] if isinstance(t, str) else int(t)


def dequant_rows(type_, w: np.ndarray, n_in: int) -> np.ndarray:
    """Dequantizes every row of the weight bytes w ([n_out][row_bytes] uint8) to f32."""
    t = _type_id(type_)
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1)
    be, bb = BLOCK[t]
    if n_in <= 0 or n_in % be:
        raise ValueError(f"n_in={n_in} is not a multiple of the block size {be}")
    row_bytes = n_in // be * bb
    n_out = w.size // row_bytes
    out = np.empty((n_out, n_in), dtype=np.float32)
    for r in range(n_out):
        rc = lib().oracle_dequant_row(t, c_void_p(w.ctypes.data + r * row_bytes),
                                      c_void_p(out[r].ctypes.data), n_in)
        if rc != 0:
            raise ValueError("oracle_dequant_row: bad argument")
    return out


def linear(type_, w: np.ndarray, x: np.ndarray, n_in: int, n_out: int, out=None, accumulate=False,
           f16_path=False, n_threads=None) -> np.ndarray:
    """out[t][r] (+)= W[r]·x[t] (ops::matvec; f16_path: the Metal batched numerics)."""
    t = _type_id(type_)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, n_in)
    n_tok = x.shape[0]
    if out is None:
        out = np.zeros((n_tok, n_out), dtype=np.float32)
    else:
        out = np.ascontiguousarray(out, dtype=np.float32).reshape(n_tok, n_out).copy()
    f = lib().oracle_linear_f16 if f16_path else lib().oracle_linear
    rc = f(t, _ptr(w), _ptr(x), _ptr(out), n_in, n_out, n_tok, 1 if accumulate else 0,
           n_threads or min(8, os.cpu_count() or 1))
    if rc != 0:
        raise ValueError("oracle_linear: bad argument")
    return out


# ---------------------------------------------------------------- model-level oracle

def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """ops::rmsnorm per row (src/ops.cpp:226-231)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    out = np.empty_like(x)
    lib().oracle_rmsnorm(_ptr(x), _ptr(np.ascontiguousarray(w, dtype=np.float32)), _ptr(out), n,
                         x.size // n, c_float(eps))
    return out


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """silu(gate) * up (src/cpu_backend.cpp:77, src/ops.h:35)."""
    g = np.ascontiguousarray(gate, dtype=np.float32).copy()
    lib().oracle_silu_mul(_ptr(g), _ptr(np.ascontiguousarray(up, dtype=np.float32)), g.size)
    return g


class _Tensor(ctypes.Structure):
    _fields_ = [("type", c_int), ("data", c_void_p)]


class _Layer(ctypes.Structure):
    _fields_ = [("attn_norm", c_void_p), ("ffn_norm", c_void_p)] + [
        (n, _Tensor) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")]


class _Model(ctypes.Structure):
    _fields_ = [(n, c_int) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff",
                                     "n_vocab")] + [
        ("rms_eps", c_float), ("rope_inv_freq", c_void_p), ("tok_embd", _Tensor), ("output", _Tensor),
        ("output_norm", c_void_p), ("layers", ctypes.POINTER(_Layer))]


class ForwardOracle:
    """CpuBackend::forward (src/cpu_backend.cpp:22-90) over a model given as numpy arrays, with an
    f16 KV cache; `forward(token, pos, f16_linear)` returns the logits."""

    def __init__(self, model, n_ctx: int, threads=None):
        self.m = model
        c = model["cfg"]
        self.n_ctx = n_ctx
        self.threads = threads or min(8, os.cpu_count() or 1)
        self._keep = []

        def arr(a, dt):
            a = np.ascontiguousarray(a, dtype=dt)
            self._keep.append(a)
            return a.ctypes.data

        def ten(t):
            return _Tensor(_type_id(t[0]), arr(t[1], np.uint8))

        layers = (_Layer * c["n_layer"])()
        for l, L in enumerate(model["layers"]):
            layers[l].attn_norm = arr(L["attn_norm"], np.float32)
            layers[l].ffn_norm = arr(L["ffn_norm"], np.float32)
            for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
                setattr(layers[l], n, ten(L[n]))
        self._layers = layers
        self.model = _Model(c["n_layer"], c["n_embd"], c["n_head"], c["n_head_kv"], c["head_dim"], c["n_ff"],
                            c["n_vocab"], c["rms_eps"], arr(model["rope_inv_freq"], np.float32),
                            ten(model["tok_embd"]), ten(model["output"]), arr(model["output_norm"], np.float32),
                            layers)
        kv_dim = c["n_head_kv"] * c["head_dim"]
        self.k_cache = np.zeros((c["n_layer"], n_ctx, kv_dim), dtype=np.uint16)
        self.v_cache = np.zeros_like(self.k_cache)
        lib().oracle_forward.argtypes = [ctypes.POINTER(_Model), c_void_p, c_void_p, c_int, c_int, c_int,
                                         c_void_p, c_int, c_int]
        lib().oracle_forward.restype = c_int

    def forward(self, token: int, pos: int, f16_linear: bool = False) -> np.ndarray:
        logits = np.empty(self.m["cfg"]["n_vocab"], dtype=np.float32)
        rc = lib().oracle_forward(ctypes.byref(self.model), _ptr(self.k_cache), _ptr(self.v_cache),
                                  self.n_ctx, token, pos, _ptr(logits), 1 if f16_linear else 0, self.threads)
        if rc != 0:
            raise ValueError("oracle_forward: bad argument")
        return logits
