"""ctypes binding of libingot_attn.so, the C ABI declared in include/ingot_attn.h and
include/ingot_linear.h.

This is the host-side mirror of the attention step of Ingot's `Backend` (src/backend.h:9-23;
the Metal dispatcher is `encode_attention`, src/metal_backend.mm:336-383). Device memory and
streams come from PyTorch (plumbing only); every computation runs in the HIP library. There is
no CPU fallback: if the library is missing or fails, these functions raise, as the reference
raises std::runtime_error (src/metal_backend.mm:421-424, 462).
"""
from __future__ import annotations

import ctypes
import math
import os
from ctypes import c_float, c_int, c_size_t, c_uint32, c_uint64, c_void_p

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libingot_attn.so")

# Exported symbols, as declared in include/ingot_attn.h and include/ingot_linear.h.
EXPORTS = (
    "ingot_attn_decode_workspace_size",
    "ingot_attn_prefill_workspace_size",
    "ingot_attn_decode_splits",
    "ingot_attn_prefill_splits",
    "ingot_attn_decode",
    "ingot_attn_decode_noalloc",
    "ingot_attn_prefill",
    "ingot_rope_kv_store",
    "ingot_attn_strerror",
    "ingot_attn_version",
    "ingot_linear_weight_bytes",
    "ingot_linear_splits",
    "ingot_linear_workspace_size",
    "ingot_linear",
    "ingot_proj",
    "ingot_proj_rope_kv",
    "ingot_rmsnorm",
    "ingot_silu_mul",
    "ingot_get_rows",
)

# GGUF tensor type ids (ggml's enum, src/gguf.h:30-33) with a linear kernel, and their
# (elements, bytes) per block (src/ops.cpp:33-87).
GGUF_TYPES = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q8_0": 8, "Q6_K": 14, "BF16": 30}
BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 8: (32, 34), 2: (32, 18), 3: (32, 20), 14: (256, 210)}


class DecodeDesc(ctypes.Structure):
    """IngotAttnDecodeDesc; mirrors AttnDecParams (src/metal_backend.mm:32)."""

    _fields_ = [
        ("n_head", c_uint32),
        ("n_head_kv", c_uint32),
        ("head_dim", c_uint32),
        ("n_keys", c_uint32),
        ("kv_offset", c_uint64),
        ("n_splits", c_uint32),
        ("scale", c_float),
    ]


class PrefillDesc(ctypes.Structure):
    """IngotAttnPrefillDesc; mirrors AttnPrefillParams (src/metal_backend.mm:33)."""

    _fields_ = [
        ("n_head", c_uint32),
        ("n_head_kv", c_uint32),
        ("head_dim", c_uint32),
        ("pos", c_uint32),
        ("n_tok", c_uint32),
        ("kv_offset", c_uint64),
        ("q_stride", c_uint32),
        ("n_splits", c_uint32),
        ("scale", c_float),
    ]


class RopeKvDesc(ctypes.Structure):
    """IngotRopeKvDesc; mirrors RopeKParams (src/metal_backend.mm:31) plus q heads and n_tok."""

    _fields_ = [
        ("n_head", c_uint32),
        ("n_head_kv", c_uint32),
        ("head_dim", c_uint32),
        ("pos", c_uint32),
        ("n_tok", c_uint32),
        ("dst_offset", c_uint64),
        ("q_stride", c_uint32),
        ("kv_stride", c_uint32),
    ]


class LinearDesc(ctypes.Structure):
    """IngotLinearDesc; mirrors MatvecParams / MatmulParams (shaders/kernels.metal:19, 716)."""

    _fields_ = [
        ("type", c_uint32),
        ("n_in", c_uint32),
        ("n_out", c_uint32),
        ("n_tok", c_uint32),
        ("out_offset", c_uint32),
        ("accumulate", c_uint32),
        ("n_splits", c_uint32),
    ]


# ingot_proj prologues and epilogues (include/ingot_linear.h).
PROJ_X, PROJ_RMSNORM = 0, 1
PROJ_STORE, PROJ_ACCUMULATE, PROJ_SILU_GATE = 0, 1, 2


class ProjDesc(ctypes.Structure):
    """IngotProjDesc: one decode token through up to three matrices sharing x, with the
    rmsnorm before and the residual add / silu gate after fused in; or (n_tok > 1) a chunk
    through up to three matrices in one batched launch (store / accumulate only)."""

    _fields_ = [
        ("type", c_uint32),
        ("n_in", c_uint32),
        ("n_mats", c_uint32),
        ("n_out", c_uint32 * 3),
        ("prologue", c_uint32),
        ("epilogue", c_uint32),
        ("eps", c_float),
        ("n_tok", c_uint32),
    ]


_lib = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads the HIP library (once). Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"libingot_attn.so not found at {path}: build it first "
            "(python -c 'import __graft_entry__ as g; g.build()')"
        )
    lib = ctypes.CDLL(path)
    PD, PP = ctypes.POINTER(DecodeDesc), ctypes.POINTER(PrefillDesc)
    lib.ingot_attn_decode_workspace_size.argtypes = [PD]
    lib.ingot_attn_decode_workspace_size.restype = c_size_t
    lib.ingot_attn_prefill_workspace_size.argtypes = [PP]
    lib.ingot_attn_prefill_workspace_size.restype = c_size_t
    lib.ingot_attn_decode_splits.argtypes = [PD]
    lib.ingot_attn_decode_splits.restype = c_uint32
    lib.ingot_attn_prefill_splits.argtypes = [PP]
    lib.ingot_attn_prefill_splits.restype = c_uint32
    lib.ingot_attn_decode.argtypes = [c_void_p] * 5 + [c_size_t, PD, c_void_p]
    lib.ingot_attn_decode.restype = c_int
    lib.ingot_attn_decode_noalloc.argtypes = [c_void_p] * 4 + [PD, c_void_p]
    lib.ingot_attn_decode_noalloc.restype = c_int
    lib.ingot_attn_prefill.argtypes = [c_void_p] * 5 + [c_size_t, PP, c_void_p]
    lib.ingot_attn_prefill.restype = c_int
    lib.ingot_rope_kv_store.argtypes = [c_void_p] * 6 + [ctypes.POINTER(RopeKvDesc), c_void_p]
    lib.ingot_rope_kv_store.restype = c_int
    lib.ingot_linear_weight_bytes.argtypes = [ctypes.POINTER(LinearDesc)]
    lib.ingot_linear_weight_bytes.restype = c_size_t
    lib.ingot_linear_splits.argtypes = [ctypes.POINTER(LinearDesc)]
    lib.ingot_linear_splits.restype = c_uint32
    lib.ingot_linear_workspace_size.argtypes = [ctypes.POINTER(LinearDesc)]
    lib.ingot_linear_workspace_size.restype = c_size_t
    lib.ingot_linear.argtypes = [c_void_p] * 4 + [c_size_t, ctypes.POINTER(LinearDesc), c_void_p]
    lib.ingot_linear.restype = c_int
    lib.ingot_proj.argtypes = [ctypes.POINTER(c_void_p), c_void_p, c_void_p, ctypes.POINTER(c_void_p),
                               ctypes.POINTER(ProjDesc), c_void_p]
    lib.ingot_proj.restype = c_int
    lib.ingot_proj_rope_kv.argtypes = [ctypes.POINTER(c_void_p), c_void_p, c_void_p] + [c_void_p] * 6 + [
        ctypes.POINTER(ProjDesc), ctypes.POINTER(RopeKvDesc), c_void_p]
    lib.ingot_proj_rope_kv.restype = c_int
    lib.ingot_rmsnorm.argtypes = [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_float, c_void_p]
    lib.ingot_rmsnorm.restype = c_int
    lib.ingot_silu_mul.argtypes = [c_void_p, c_void_p, c_uint64, c_void_p]
    lib.ingot_silu_mul.restype = c_int
    lib.ingot_get_rows.argtypes = [c_uint32, c_void_p, c_uint32, c_uint32, c_void_p, c_uint32, c_void_p,
                                   c_void_p]
    lib.ingot_get_rows.restype = c_int
    lib.ingot_attn_strerror.argtypes = [c_int]
    lib.ingot_attn_strerror.restype = ctypes.c_char_p
    lib.ingot_attn_version.argtypes = []
    lib.ingot_attn_version.restype = ctypes.c_char_p
    _lib = lib
    return lib


def decode_desc(n_head, n_head_kv, head_dim, n_keys, kv_offset=0, n_splits=0, scale=None):
    scale = 1.0 / math.sqrt(head_dim) if scale is None else scale
    return DecodeDesc(n_head, n_head_kv, head_dim, n_keys, kv_offset, n_splits, scale)


def prefill_desc(n_head, n_head_kv, head_dim, pos, n_tok, kv_offset=0, q_stride=None, n_splits=0,
                 scale=None):
    scale = 1.0 / math.sqrt(head_dim) if scale is None else scale
    q_stride = n_head * head_dim if q_stride is None else q_stride
    return PrefillDesc(n_head, n_head_kv, head_dim, pos, n_tok, kv_offset, q_stride, n_splits, scale)


def rope_kv_desc(n_head, n_head_kv, head_dim, pos, n_tok, dst_offset=0, q_stride=None,
                 kv_stride=None):
    q_stride = n_head * head_dim if q_stride is None else q_stride
    kv_stride = n_head_kv * head_dim if kv_stride is None else kv_stride
    return RopeKvDesc(n_head, n_head_kv, head_dim, pos, n_tok, dst_offset, q_stride, kv_stride)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load_library().ingot_attn_strerror(rc).decode()
        raise RuntimeError(f"{what} failed: {msg} (code {rc})")


class Workspace:
    """A zero-initialised device workspace that grows on demand (never shrinks).

    The library leaves its completion counters at zero after every call, so the buffer is
    zeroed only when (re)allocated.
    """

    def __init__(self, device="cuda"):
        self.device = device
        self.buf = None

    def get(self, nbytes: int):
        import torch

        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=self.device)
        return self.buf


_default_ws = {}


def _workspace(device):
    key = str(device)
    if key not in _default_ws:
        _default_ws[key] = Workspace(device)
    return _default_ws[key]


def _stream_ptr(stream):
    import torch

    s = torch.cuda.current_stream() if stream is None else stream
    return c_void_p(s.cuda_stream)


def attn_decode(q, k_cache, v_cache, out, desc: DecodeDesc, stream=None, workspace=None):
    """One decode step: out[n_head*hd] = attention of q over cache rows 0..n_keys-1.

    q, out: f32 CUDA tensors; k_cache, v_cache: f16 (or int16/uint16 bit-views) CUDA tensors
    holding the [layer][n_ctx][n_head_kv*hd] cache. Launches on `stream` (default: torch's
    current stream) and returns without synchronizing.
    """
    lib = load_library()
    nbytes = lib.ingot_attn_decode_workspace_size(ctypes.byref(desc))
    if nbytes == 0:
        _check(-1, "ingot_attn_decode_workspace_size")
    ws = (workspace or _workspace(q.device)).get(nbytes)
    rc = lib.ingot_attn_decode(
        c_void_p(q.data_ptr()), c_void_p(k_cache.data_ptr()), c_void_p(v_cache.data_ptr()),
        c_void_p(out.data_ptr()), c_void_p(ws.data_ptr()), c_size_t(ws.numel()),
        ctypes.byref(desc), _stream_ptr(stream))
    _check(rc, "ingot_attn_decode")
    return out


def attn_decode_noalloc(q, k_cache, v_cache, out, desc: DecodeDesc, stream=None):
    """ingot_attn_decode_noalloc: the same decode step on the library's device-resident scratch
    (no workspace argument, no allocation)."""
    rc = load_library().ingot_attn_decode_noalloc(
        c_void_p(q.data_ptr()), c_void_p(k_cache.data_ptr()), c_void_p(v_cache.data_ptr()),
        c_void_p(out.data_ptr()), ctypes.byref(desc), _stream_ptr(stream))
    _check(rc, "ingot_attn_decode_noalloc")
    return out


def attn_prefill(q, k_cache, v_cache, out, desc: PrefillDesc, stream=None, workspace=None):
    """Causal prefill of desc.n_tok queries at positions desc.pos.. over the cache."""
    lib = load_library()
    nbytes = lib.ingot_attn_prefill_workspace_size(ctypes.byref(desc))
    if nbytes == 0:
        _check(-1, "ingot_attn_prefill_workspace_size")
    ws = (workspace or _workspace(q.device)).get(nbytes)
    rc = lib.ingot_attn_prefill(
        c_void_p(q.data_ptr()), c_void_p(k_cache.data_ptr()), c_void_p(v_cache.data_ptr()),
        c_void_p(out.data_ptr()), c_void_p(ws.data_ptr()), c_size_t(ws.numel()),
        ctypes.byref(desc), _stream_ptr(stream))
    _check(rc, "ingot_attn_prefill")
    return out


def decode_splits(desc: DecodeDesc) -> int:
    return int(load_library().ingot_attn_decode_splits(ctypes.byref(desc)))


def prefill_splits(desc: PrefillDesc) -> int:
    return int(load_library().ingot_attn_prefill_splits(ctypes.byref(desc)))


def rope_kv_store(q, k, v, k_cache, v_cache, inv_freq, desc: RopeKvDesc, stream=None):
    """RoPE on q (in place; None to skip) and k, K and V into the f16 cache rows, one launch.

    q, k, v, inv_freq: f32 CUDA tensors; k_cache, v_cache: f16 (or 16-bit views) CUDA tensors.
    Replaces the reference's rope + rope_k_to_cache + to_half (src/metal_backend.mm:395-409).
    """
    lib = load_library()
    rc = lib.ingot_rope_kv_store(
        None if q is None else c_void_p(q.data_ptr()), c_void_p(k.data_ptr()),
        c_void_p(v.data_ptr()), c_void_p(k_cache.data_ptr()), c_void_p(v_cache.data_ptr()),
        c_void_p(inv_freq.data_ptr()), ctypes.byref(desc), _stream_ptr(stream))
    _check(rc, "ingot_rope_kv_store")


def linear_desc(type_, n_in, n_out, n_tok=1, out_offset=0, accumulate=False, n_splits=0):
    t = GGUF_TYPES[type_] if isinstance(type_, str) else int(type_)
    return LinearDesc(t, n_in, n_out, n_tok, out_offset, 1 if accumulate else 0, n_splits)


def linear_splits(desc: LinearDesc) -> int:
    return int(load_library().ingot_linear_splits(ctypes.byref(desc)))


def linear_weight_bytes(desc: LinearDesc) -> int:
    return int(load_library().ingot_linear_weight_bytes(ctypes.byref(desc)))


def linear_workspace_size(desc: LinearDesc) -> int:
    return int(load_library().ingot_linear_workspace_size(ctypes.byref(desc)))


def linear(w, x, out, desc: LinearDesc, stream=None, workspace=None, use_workspace=True):
    """out[out_offset + t*n_out + r] (+)= W[r]·x[t] over the GGUF weight bytes `w`.

    w: uint8 CUDA tensor of the raw weight bytes (ingot_linear_weight_bytes long); x, out: f32
    CUDA tensors. Replaces encode_linear (src/metal_backend.mm:282-310); with accumulate it is
    the wo projection plus residual add (src/metal_backend.mm:446-447). The workspace (shared
    per device by default) lets small batched calls split over n_in; use_workspace=False runs
    without one.
    """
    lib = load_library()
    ws, nws = None, 0
    if use_workspace:
        nbytes = lib.ingot_linear_workspace_size(ctypes.byref(desc))
        if nbytes == 0:
            _check(-1, "ingot_linear_workspace_size")
        buf = (workspace or _workspace(x.device)).get(nbytes)
        ws, nws = c_void_p(buf.data_ptr()), buf.numel()
    rc = lib.ingot_linear(c_void_p(w.data_ptr()), c_void_p(x.data_ptr()), c_void_p(out.data_ptr()),
                          ws, c_size_t(nws), ctypes.byref(desc), _stream_ptr(stream))
    _check(rc, "ingot_linear")
    return out


def proj_desc(type_, n_in, n_out, prologue=PROJ_X, epilogue=PROJ_STORE, eps=0.0, n_tok=1):
    t = GGUF_TYPES[type_] if isinstance(type_, str) else int(type_)
    n_out = list(n_out)
    return ProjDesc(t, n_in, len(n_out), (c_uint32 * 3)(*(n_out + [0] * (3 - len(n_out)))),
                    prologue, epilogue, eps, n_tok)


def proj(ws, x, outs, desc: ProjDesc, norm_w=None, stream=None):
    """One token (or a chunk, desc.n_tok > 1): out[m] (+)= W[m]·x' for the weight-byte tensors `ws`, x' = x or
    rmsnorm(x) * norm_w; with PROJ_SILU_GATE (ws = [gate, up]) outs[0] = silu(gate·x') * (up·x').
    The fused form of rmsnorm + encode_linear (+ encode_silu_mul) (src/metal_backend.mm:433-452)."""
    n = len(ws)
    wp = (c_void_p * n)(*[w.data_ptr() for w in ws])
    op = (c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    rc = load_library().ingot_proj(wp, c_void_p(x.data_ptr()),
                                   c_void_p(norm_w.data_ptr() if norm_w is not None else 0), op,
                                   ctypes.byref(desc), _stream_ptr(stream))
    _check(rc, "ingot_proj")
    return outs


def proj_rope_kv(ws, x, q, k, v, k_cache, v_cache, inv_freq, desc: ProjDesc, rope: "RopeKvDesc",
                 norm_w=None, stream=None):
    """One decode token: (rmsnorm +) q/k/v projections, RoPE on q and k, K/V into the cache rows
    (ingot_proj_rope_kv; k and v are scratch)."""
    wp = (c_void_p * 3)(*[w.data_ptr() for w in ws])
    rc = load_library().ingot_proj_rope_kv(
        wp, c_void_p(x.data_ptr()), c_void_p(norm_w.data_ptr() if norm_w is not None else 0),
        c_void_p(q.data_ptr()), c_void_p(k.data_ptr()), c_void_p(v.data_ptr()),
        c_void_p(k_cache.data_ptr()), c_void_p(v_cache.data_ptr()), c_void_p(inv_freq.data_ptr()),
        ctypes.byref(desc), ctypes.byref(rope), _stream_ptr(stream))
    _check(rc, "ingot_proj_rope_kv")
    return q


def rmsnorm(x, w, out, n, n_rows, eps, stream=None):
    """out = rmsnorm(x) * w per row (include/ingot_model.h; encode_rmsnorm)."""
    rc = load_library().ingot_rmsnorm(c_void_p(x.data_ptr()), c_void_p(w.data_ptr()), c_void_p(out.data_ptr()),
                                      n, n_rows, c_float(eps), _stream_ptr(stream))
    _check(rc, "ingot_rmsnorm")
    return out


def silu_mul(gate, up, n, stream=None):
    """gate = silu(gate) * up (encode_silu_mul)."""
    rc = load_library().ingot_silu_mul(c_void_p(gate.data_ptr()), c_void_p(up.data_ptr()), n,
                                       _stream_ptr(stream))
    _check(rc, "ingot_silu_mul")
    return gate


def get_rows(type_, w, n, n_rows, tokens, n_tok, out, stream=None):
    """out[t] = dequantized row tokens[t] of the GGUF table w (tokens: int32 CUDA tensor)."""
    t = GGUF_TYPES[type_] if isinstance(type_, str) else int(type_)
    rc = load_library().ingot_get_rows(t, c_void_p(w.data_ptr()), n, n_rows, c_void_p(tokens.data_ptr()),
                                       n_tok, c_void_p(out.data_ptr()), _stream_ptr(stream))
    _check(rc, "ingot_get_rows")
    return out
