"""Writes tests/golden/*.npz: seeded regression fixtures produced by this repository's CPU
oracle (oracle/attn_oracle.cpp). They are NOT reference outputs (the reference ships no
attention vectors and cannot be built here); they freeze the pinned oracle's results so that a
later change to the oracle, the input generator or a kernel shows up as a diff.

    python tests/golden/gen_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "inference-agent_amd"))
import oracle_lib  # noqa: E402
import workloads as W  # noqa: E402


def small(seed, n_head, n_head_kv, pos, n_tok, n_ctx):
    rng = np.random.Generator(np.random.PCG64(seed))
    L = pos + n_tok
    q = rng.standard_normal((n_tok, n_head * 128)).astype(np.float32)
    kb = (rng.standard_normal((n_ctx, n_head_kv * 128))).astype(np.float16).view(np.uint16)
    vb = (rng.standard_normal((n_ctx, n_head_kv * 128))).astype(np.float16).view(np.uint16)
    out = oracle_lib.attn_prefill(q, kb, vb, n_head, n_head_kv, 128, pos, n_tok)
    return dict(q=q, k=kb, v=vb, out=out, n_head=n_head, n_head_kv=n_head_kv, pos=pos, n_tok=n_tok)


def kv_store(seed, n_head, n_head_kv, pos, n_tok, n_ctx, theta):
    """RoPE + f16 KV store of n_tok tokens at pos into layer 1 of a 2-layer cache."""
    rng = np.random.Generator(np.random.PCG64(seed))
    hd = 128
    inv = oracle_lib.rope_inv_freq(theta, hd)
    q = rng.standard_normal((n_tok, n_head * hd)).astype(np.float32)
    k = rng.standard_normal((n_tok, n_head_kv * hd)).astype(np.float32)
    v = rng.standard_normal((n_tok, n_head_kv * hd)).astype(np.float32)
    cache = np.zeros((2 * n_ctx, n_head_kv * hd), dtype=np.uint16)
    dst = (n_ctx + pos) * n_head_kv * hd
    q_out, kc, vc = oracle_lib.rope_kv_store(q, k, v, cache, cache, dst, n_head, n_head_kv, hd, pos, inv)
    rows = slice(n_ctx + pos, n_ctx + pos + n_tok)
    return dict(q=q, k=k, v=v, inv_freq=inv, q_out=q_out, k_rows=kc[rows], v_rows=vc[rows],
                n_head=n_head, n_head_kv=n_head_kv, pos=pos, n_tok=n_tok, n_ctx=n_ctx)


def main():
    np.savez_compressed(os.path.join(HERE, "small_decode_g3.npz"), **small(101, 6, 2, 69, 1, 70))
    np.savez_compressed(os.path.join(HERE, "small_prefill_g3.npz"), **small(102, 6, 2, 20, 37, 57))
    np.savez_compressed(os.path.join(HERE, "small_prefill_g2.npz"), **small(103, 4, 2, 0, 65, 65))
    # Full-size configs: inputs are regenerated from the seed (numpy PCG64); the fixture keeps
    # a digest of the inputs and the oracle output.
    for w in (W.C1, W.C3):
        q, kb, vb = W.make_inputs(w)
        digest = hashlib.sha256(q.tobytes() + kb.tobytes() + vb.tobytes()).hexdigest()
        out = oracle_lib.attn_decode(q, kb, vb, 24, 8, 128, w.n_keys, threads=8)
        np.savez_compressed(os.path.join(HERE, f"{w.name}.npz"), out=out, digest=np.array(digest))
    np.savez_compressed(os.path.join(HERE, "small_kv_store.npz"), **kv_store(104, 24, 8, 2000, 5, 2048, 500000.0))
    print("written")


if __name__ == "__main__":
    main()
