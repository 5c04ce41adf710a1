"""The Llama forward pass on the MI355X through the C ABI: the Python mirror of the C++ host
class `ingot::HipBackend` (host/ingot_hip_backend.hpp), used by the tests and the bench.

Follows `MetalBackend::forward_batch` (src/metal_backend.mm:419-471) step by step: embedding
rows; per layer rmsnorm, q/k/v projections, RoPE + KV-cache store, attention, wo with the
residual add, rmsnorm, gate/up projections, silu_mul, down with the residual add; the final
rmsnorm of the last token and the logits projection. For one token (decode) the rmsnorm, the
q/k/v projections, RoPE and the KV store are one `ingot_proj_rope_kv` call, rmsnorm + gate/up +
silu_mul and the final rmsnorm + logits one `ingot_proj` launch each (identical results, fewer
launches); for a chunk large enough, q/k/v are one batched launch and gate/up + silu_mul another.
Every step is one libingot_attn.so call; PyTorch only holds device memory and the stream. Errors are the reference's
(src/metal_backend.mm:421-424): "… batch size out of range", "context window exceeded",
"token id out of range".
"""
from __future__ import annotations

import math

import numpy as np

import ingot_attn as ia


# Tiles (256 rows x 64 tokens over q, k and v) from which a chunk's q/k/v run as one batched
# launch; a test sets 0 to force that path.
QKV_ONE_LAUNCH_MIN_TILES = 128


def qkv_one_launch(n_tok, q_dim, kv_dim):
    """Whether a chunk's q/k/v run as one batched launch (ingot_proj, no split-K) rather than
    three ingot_linear calls (each split-K over the 256 CUs): when the three matrices' tiles of
    256 rows x 64 tokens reach half the CUs together (Llama-3.2-3B at 512 tokens: 160 tiles; at
    256 tokens 80, where three split launches are faster)."""
    rows = -(-q_dim // 256) + 2 * -(-kv_dim // 256)
    return rows * -(-n_tok // 64) >= QKV_ONE_LAUNCH_MIN_TILES


# Tiles (128 rows of gate and of up x 64 tokens) from which a chunk's gate/up + silu run as one
# batched launch; a test sets 0 to force that path.
FFN_ONE_LAUNCH_MIN_TILES = 256


def ffn_one_launch(n_tok, n_ff):
    """Whether a chunk's gate and up projections and silu(gate) * up run as one batched launch
    (ingot_proj with the silu epilogue, no split-K) rather than two ingot_linear calls (each
    split-K over the CUs when its tiles are few) and ingot_silu_mul: once the paired tiles fill
    the 256 CUs (Llama-3.2-3B: 512 tiles at 512 tokens, 256 at 256)."""
    return -(-n_ff // 128) * -(-n_tok // 64) >= FFN_ONE_LAUNCH_MIN_TILES


class HipForward:
    def __init__(self, model: dict, n_ctx: int, n_batch: int, device="cuda:0"):
        import torch

        c = model["cfg"]
        self.c, self.n_ctx, self.n_batch = c, n_ctx, n_batch
        dev = torch.device(device)
        self.dev = dev
        hd = c["head_dim"]
        self.q_dim, self.kv_dim = c["n_head"] * hd, c["n_head_kv"] * hd

        def up_t(t):  # (type, bytes) -> (type, device uint8 tensor)
            return (t[0], torch.from_numpy(np.ascontiguousarray(t[1]).reshape(-1)).to(dev))

        def up_f(a):
            return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)

        self.tok_embd = up_t(model["tok_embd"])
        self.output = self.tok_embd if model["output"] is model["tok_embd"] else up_t(model["output"])
        self.output_norm = up_f(model["output_norm"])
        self.inv_freq = up_f(model["rope_inv_freq"])
        self.layers = [{k: (up_f(v) if k.endswith("norm") else up_t(v)) for k, v in L.items()}
                       for L in model["layers"]]
        f32 = dict(dtype=torch.float32, device=dev)
        self.k_cache = torch.zeros(c["n_layer"] * n_ctx, self.kv_dim, dtype=torch.float16, device=dev)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.x = torch.zeros(n_batch, c["n_embd"], **f32)
        self.h = torch.zeros(n_batch, c["n_embd"], **f32)
        self.q = torch.zeros(n_batch, self.q_dim, **f32)
        self.k = torch.zeros(n_batch, self.kv_dim, **f32)
        self.v = torch.zeros(n_batch, self.kv_dim, **f32)
        self.attn = torch.zeros(n_batch, self.q_dim, **f32)
        self.gate = torch.zeros(n_batch, c["n_ff"], **f32)
        self.up = torch.zeros(n_batch, c["n_ff"], **f32)
        self.logits = torch.zeros(c["n_vocab"], **f32)
        self.tokens = torch.zeros(n_batch, dtype=torch.int32, device=dev)
        self.attn_ws = ia.Workspace(dev)
        self.lin_ws = ia.Workspace(dev)
        self.scale = 1.0 / math.sqrt(hd)

    def _lin(self, w, x, out, n_in, n_out, n, acc=False, out_offset=0):
        ia.linear(w[1], x, out, ia.linear_desc(w[0], n_in, n_out, n, out_offset=out_offset, accumulate=acc),
                  workspace=self.lin_ws)

    def forward_batch(self, tokens, pos: int, tokens_on_device=None):
        """Runs tokens at positions pos..pos+n-1; returns the logits after the last one (a
        device tensor owned by this object). `tokens_on_device` (int32 CUDA tensor of the same
        ids) skips the host-to-device copy, e.g. under graph capture."""
        import torch

        c = self.c
        n = len(tokens)
        if n < 1 or n > self.n_batch:
            raise RuntimeError("hip: batch size out of range")
        if pos < 0 or pos + n > self.n_ctx:
            raise RuntimeError("context window exceeded")
        for t in tokens:
            if t < 0 or t >= c["n_vocab"]:
                raise RuntimeError("token id out of range")
        if tokens_on_device is None:
            self.tokens[:n].copy_(torch.as_tensor(np.asarray(tokens, dtype=np.int32)))
            tok = self.tokens
        else:
            tok = tokens_on_device
        ne, qd, kvd, nf = c["n_embd"], self.q_dim, self.kv_dim, c["n_ff"]
        E = self.tok_embd
        ia.get_rows(E[0], E[1], ne, c["n_vocab"], tok, n, self.x)
        eps = c["rms_eps"]
        for l, L in enumerate(self.layers):
            rope = ia.rope_kv_desc(c["n_head"], c["n_head_kv"], c["head_dim"], pos, n,
                                   dst_offset=(l * self.n_ctx + pos) * kvd)
            if n == 1 and L["wq"][0] == L["wk"][0] == L["wv"][0]:
                ia.proj_rope_kv([L["wq"][1], L["wk"][1], L["wv"][1]], self.x, self.q, self.k, self.v,
                                self.k_cache, self.v_cache, self.inv_freq,
                                ia.proj_desc(L["wq"][0], ne, [qd, kvd, kvd], prologue=ia.PROJ_RMSNORM, eps=eps),
                                rope, norm_w=L["attn_norm"])
            else:
                ia.rmsnorm(self.x, L["attn_norm"], self.h, ne, n, eps)
                if n > 1 and L["wq"][0] == L["wk"][0] == L["wv"][0] and qkv_one_launch(n, qd, kvd):
                    ia.proj([L["wq"][1], L["wk"][1], L["wv"][1]], self.h, [self.q, self.k, self.v],
                            ia.proj_desc(L["wq"][0], ne, [qd, kvd, kvd], n_tok=n))
                else:
                    self._lin(L["wq"], self.h, self.q, ne, qd, n)
                    self._lin(L["wk"], self.h, self.k, ne, kvd, n)
                    self._lin(L["wv"], self.h, self.v, ne, kvd, n)
                ia.rope_kv_store(self.q, self.k, self.v, self.k_cache, self.v_cache, self.inv_freq, rope)
            kv_offset = l * self.n_ctx * kvd
            if n == 1:
                ia.attn_decode(self.q, self.k_cache, self.v_cache, self.attn,
                               ia.decode_desc(c["n_head"], c["n_head_kv"], c["head_dim"], pos + 1,
                                              kv_offset=kv_offset, scale=self.scale), workspace=self.attn_ws)
            else:
                ia.attn_prefill(self.q, self.k_cache, self.v_cache, self.attn,
                                ia.prefill_desc(c["n_head"], c["n_head_kv"], c["head_dim"], pos, n,
                                                kv_offset=kv_offset, scale=self.scale), workspace=self.attn_ws)
            self._lin(L["wo"], self.attn, self.x, qd, ne, n, acc=True)
            if n == 1 and L["w_gate"][0] == L["w_up"][0]:
                ia.proj([L["w_gate"][1], L["w_up"][1]], self.x, [self.gate],
                        ia.proj_desc(L["w_gate"][0], ne, [nf, nf], prologue=ia.PROJ_RMSNORM,
                                     epilogue=ia.PROJ_SILU_GATE, eps=eps),
                        norm_w=L["ffn_norm"])
            elif L["w_gate"][0] == L["w_up"][0] and ffn_one_launch(n, nf):
                ia.rmsnorm(self.x, L["ffn_norm"], self.h, ne, n, eps)
                ia.proj([L["w_gate"][1], L["w_up"][1]], self.h, [self.gate],
                        ia.proj_desc(L["w_gate"][0], ne, [nf, nf], epilogue=ia.PROJ_SILU_GATE, n_tok=n))
            else:
                ia.rmsnorm(self.x, L["ffn_norm"], self.h, ne, n, eps)
                self._lin(L["w_gate"], self.h, self.gate, ne, nf, n)
                self._lin(L["w_up"], self.h, self.up, ne, nf, n)
                ia.silu_mul(self.gate, self.up, n * nf)
            self._lin(L["w_down"], self.gate, self.x, nf, ne, n, acc=True)
        # logits for the last token only (src/metal_backend.mm:454-456)
        last = self.x[n - 1:n]
        O = self.output
        ia.proj([O[1]], last, [self.logits],
                ia.proj_desc(O[0], ne, [c["n_vocab"]], prologue=ia.PROJ_RMSNORM, eps=eps),
                norm_w=self.output_norm)
        return self.logits

    def forward(self, token: int, pos: int):
        return self.forward_batch([token], pos)
