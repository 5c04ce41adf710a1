"""GPU parity of the fused one-token projection (ingot_proj) — the rmsnorm before q/k/v and
gate/up, up to three matrices in one launch, the residual accumulate and the silu gate after.

Two bars, stated per test:
  - against the unfused library sequence (ingot_rmsnorm, ingot_linear with n_tok = 1,
    ingot_silu_mul): bit-exact — the fused kernel performs the same f32 operations in the same
    order;
  - against the CPU oracle (ops::rmsnorm, ops::matvec, silu(gate)*up): rel-L2 <= 1e-5 and
    max|d| <= 1e-5 * max|ref| + 1e-6, the bar of the linear layer's one-token path (the order of
    the f32 sums differs, and the GPU's expf in the silu).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import ensure_built

import gguf_blocks as gb

pytestmark = pytest.mark.gpu

TYPES = ["F32", "F16", "BF16", "Q8_0", "Q4_0", "Q4_1", "Q6_K"]
EPS = 1e-5


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


def _close(got, want, what):
    d = np.abs(got.astype(np.float64) - want)
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    tol = 1e-5 * np.abs(want).max() + 1e-6
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert d.max() <= tol and rel <= 1e-5, f"{what}: max|d|={d.max():.3e} (tol {tol:.1e}), rel-L2={rel:.3e}"


def _inputs(t, n_in, n_outs, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((1, n_in)) * 2).astype(np.float32)
    nw = (1 + 0.3 * rng.standard_normal(n_in)).astype(np.float32)
    raws = [gb.random_weights(t, n, n_in, seed=seed + 10 * i + 1) for i, n in enumerate(n_outs)]
    return x, nw, raws


def _unfused(dev, t, raws, x, nw, n_in, n_outs, rms, base=None):
    """The same step as separate library calls: rmsnorm, one ingot_linear per matrix."""
    import torch
    import ingot_attn as ia

    xd = _t(x, dev)
    h = torch.empty_like(xd)
    if rms:
        ia.rmsnorm(xd, _t(nw, dev), h, n_in, 1, EPS)
    else:
        h = xd
    outs = []
    for i, (raw, n) in enumerate(zip(raws, n_outs)):
        out = _t(base[i] if base is not None else np.zeros((1, n), np.float32), dev)
        ia.linear(_t(raw.reshape(-1), dev), h, out, ia.linear_desc(t, n_in, n, 1, accumulate=base is not None),
                  use_workspace=False)
        outs.append(out)
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_in,n_outs", [(3072, (3072, 1024, 1024)), (512, (200, 77, 3)), (256, (1001,))])
def test_rmsnorm_qkv(dev, oracle_mod, t, n_in, n_outs):
    import torch
    import ingot_attn as ia

    x, nw, raws = _inputs(t, n_in, n_outs, seed=n_in + len(n_outs))
    outs = [_t(np.full((1, n), np.nan, np.float32), dev) for n in n_outs]
    d = ia.proj_desc(t, n_in, n_outs, prologue=ia.PROJ_RMSNORM, eps=EPS)
    ia.proj([_t(r.reshape(-1), dev) for r in raws], _t(x, dev), outs, d, norm_w=_t(nw, dev))
    torch.cuda.synchronize()
    ref = _unfused(dev, t, raws, x, nw, n_in, n_outs, rms=True)
    h = oracle_mod.rmsnorm(x, nw, EPS)
    for i, (o, r, raw, n) in enumerate(zip(outs, ref, raws, n_outs)):
        got = o.cpu().numpy()
        assert np.array_equal(got, r.cpu().numpy()), f"{t} matrix {i}: fused != rmsnorm + ingot_linear"
        _close(got, oracle_mod.linear(t, raw, h, n_in, n), f"{t} {n_in}x{n} matrix {i}")


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_in,n_ff", [(3072, 8192), (512, 1000), (256, 5)])
def test_rmsnorm_gate_up_silu(dev, oracle_mod, t, n_in, n_ff):
    import torch
    import ingot_attn as ia

    x, nw, raws = _inputs(t, n_in, (n_ff, n_ff), seed=7 + n_ff)
    out = _t(np.full((1, n_ff), np.nan, np.float32), dev)
    d = ia.proj_desc(t, n_in, [n_ff, n_ff], prologue=ia.PROJ_RMSNORM, epilogue=ia.PROJ_SILU_GATE, eps=EPS)
    ia.proj([_t(r.reshape(-1), dev) for r in raws], _t(x, dev), [out], d, norm_w=_t(nw, dev))
    torch.cuda.synchronize()
    g, u = _unfused(dev, t, raws, x, nw, n_in, (n_ff, n_ff), rms=True)
    ia.silu_mul(g, u, n_ff) if n_ff % 4 == 0 else None
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    if n_ff % 4 == 0:  # ingot_silu_mul takes multiples of 4
        assert np.array_equal(got, g.cpu().numpy()), f"{t}: fused != rmsnorm + linear x2 + silu_mul"
    h = oracle_mod.rmsnorm(x, nw, EPS)
    want = oracle_mod.silu_mul(oracle_mod.linear(t, raws[0], h, n_in, n_ff),
                               oracle_mod.linear(t, raws[1], h, n_in, n_ff))
    _close(got, want, f"{t} gate/up {n_in}x{n_ff}")


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_in,n_out", [(3072, 3072), (8192, 3072), (512, 37)])
def test_accumulate(dev, oracle_mod, t, n_in, n_out):
    """wo / w_down: out += W·x, no prologue."""
    import torch
    import ingot_attn as ia

    x, nw, raws = _inputs(t, n_in, (n_out,), seed=3 + n_in)
    base = np.random.default_rng(9).standard_normal((1, n_out)).astype(np.float32)
    out = _t(base, dev)
    ia.proj([_t(raws[0].reshape(-1), dev)], _t(x, dev), [out],
            ia.proj_desc(t, n_in, [n_out], epilogue=ia.PROJ_ACCUMULATE))
    torch.cuda.synchronize()
    ref = _unfused(dev, t, raws, x, nw, n_in, (n_out,), rms=False, base=[base])[0]
    got = out.cpu().numpy()
    assert np.array_equal(got, ref.cpu().numpy()), f"{t}: fused != ingot_linear accumulate"
    _close(got, base + oracle_mod.linear(t, raws[0], x, n_in, n_out), f"{t} accumulate {n_in}x{n_out}")


def test_rows_too_long(dev):
    """Rows whose staging exceeds the 160 KB of LDS are refused, not truncated."""
    import torch
    import ingot_attn as ia

    n_in = 32768  # x alone is 128 KB; with the rmsnorm weights 256 KB
    w = torch.zeros(n_in // 32 * 18 * 4, dtype=torch.uint8, device=dev)
    x = torch.zeros(n_in, device=dev)
    out = torch.zeros(4, device=dev)
    with pytest.raises(RuntimeError):
        ia.proj([w], x, [out], ia.proj_desc("Q4_0", n_in, [4], prologue=ia.PROJ_RMSNORM, eps=EPS), norm_w=x)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("pos", [0, 1, 777, 4095])
def test_proj_rope_kv(dev, t, pos):
    """rmsnorm + q/k/v + RoPE + KV store in one call equals ingot_proj (store) followed by
    ingot_rope_kv_store, bit for bit: q, the written K/V cache rows, and every other cache row
    keeps its canary bits."""
    import torch
    import ingot_attn as ia

    n_head, n_head_kv, hd, n_in, n_ctx = 24, 8, 128, 3072, 4096 + 8
    qd, kvd = n_head * hd, n_head_kv * hd
    x, nw, raws = _inputs(t, n_in, (qd, kvd, kvd), seed=11 + pos)
    wd = [_t(r.reshape(-1), dev) for r in raws]
    inv = torch.tensor([500000.0 ** (-2 * i / hd) for i in range(hd // 2)], dtype=torch.float32, device=dev)
    canary = torch.full((n_ctx, kvd), 0x7E00, dtype=torch.int16, device=dev).view(torch.float16)
    desc = ia.proj_desc(t, n_in, [qd, kvd, kvd], prologue=ia.PROJ_RMSNORM, eps=EPS)
    rope = ia.rope_kv_desc(n_head, n_head_kv, hd, pos, 1, dst_offset=pos * kvd)
    # fused
    q1, k1, v1 = (torch.zeros(n, device=dev) for n in (qd, kvd, kvd))
    kc1, vc1 = canary.clone(), canary.clone()
    ia.proj_rope_kv(wd, _t(x, dev), q1, k1, v1, kc1, vc1, inv, desc, rope, norm_w=_t(nw, dev))
    # two calls
    q2, k2, v2 = (torch.zeros(n, device=dev) for n in (qd, kvd, kvd))
    kc2, vc2 = canary.clone(), canary.clone()
    ia.proj(wd, _t(x, dev), [q2, k2, v2], desc, norm_w=_t(nw, dev))
    ia.rope_kv_store(q2, k2, v2, kc2, vc2, inv, rope)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2), f"{t} pos {pos}: q differs"
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16)), f"{t} pos {pos}: K cache differs"
    assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16)), f"{t} pos {pos}: V cache differs"
    untouched = torch.ones(n_ctx, dtype=torch.bool, device=dev)
    untouched[pos] = False
    assert bool((kc1.view(torch.int16)[untouched] == 0x7E00).all())
    assert bool((vc1.view(torch.int16)[untouched] == 0x7E00).all())


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_tok,n_in,n_outs,acc", [(512, 3072, (3072, 1024, 1024), False),
                                                   (70, 512, (200, 77, 3), False),
                                                   (130, 768, (257, 513), True)])
def test_chunk_matrices_one_launch(dev, oracle_mod, t, n_tok, n_in, n_outs, acc):
    """A chunk (n_tok > 1) through up to three matrices in one batched launch: each output
    equals ingot_linear on its matrix (same n_tok, n_splits = 1) bit for bit, the f16-rounding
    oracle (oracle_linear_f16) on sampled token rows within the matmul bar (rel-L2 <= 1e-5,
    max|d| <= 1e-5 * max|ref| + 1e-6), and nothing past a matrix's [n_tok][n_out] is written."""
    import torch
    import ingot_attn as ia

    rng = np.random.default_rng(n_tok + n_in)
    x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
    raws = [gb.random_weights(t, n, n_in, seed=n_in + 7 * i + 1) for i, n in enumerate(n_outs)]
    bases = [rng.standard_normal((n_tok, n)).astype(np.float32) if acc else None for n in n_outs]
    pad = 29

    def fresh(i):
        buf = np.full(n_tok * n_outs[i] + pad, np.nan, np.float32)
        if acc:
            buf[: n_tok * n_outs[i]] = bases[i].ravel()
        return _t(buf, dev)

    xd = _t(x, dev)
    wd = [_t(r.reshape(-1), dev) for r in raws]
    outs = [fresh(i) for i in range(len(n_outs))]
    ia.proj(wd, xd, outs, ia.proj_desc(t, n_in, list(n_outs), epilogue=ia.PROJ_ACCUMULATE if acc else ia.PROJ_STORE,
                                       n_tok=n_tok))
    refs = [fresh(i) for i in range(len(n_outs))]
    for w, r, n in zip(wd, refs, n_outs):
        ia.linear(w, xd, r, ia.linear_desc(t, n_in, n, n_tok, accumulate=acc, n_splits=1), use_workspace=False)
    torch.cuda.synchronize()
    rows = sorted({0, 1, n_tok // 2, n_tok - 2, n_tok - 1})
    for i, (o, r, raw, n) in enumerate(zip(outs, refs, raws, n_outs)):
        got = o.cpu().numpy()
        assert np.array_equal(got, r.cpu().numpy(), equal_nan=True), f"{t} matrix {i}: != ingot_linear"
        assert np.all(np.isnan(got[n_tok * n:])), f"{t} matrix {i}: wrote past its rows"
        got = got[: n_tok * n].reshape(n_tok, n)[rows]
        base = bases[i][rows] if acc else None
        want = oracle_mod.linear(t, raw, x[rows], n_in, n, out=base, accumulate=acc, f16_path=True)
        _close(got, want, f"{t} chunk {n_tok}x{n_in}x{n} matrix {i}")


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_tok,n_in,n_ff", [(512, 3072, 8192), (70, 512, 200), (130, 768, 257)])
def test_chunk_gate_up_silu(dev, oracle_mod, t, n_tok, n_in, n_ff):
    """A chunk's gate/up projections with the silu epilogue in one launch (128 rows of each
    matrix per tile): equal bit for bit to ingot_linear on gate and on up (n_splits = 1) followed
    by ingot_silu_mul, within the matmul bar of the f16-rounding oracle on sampled rows, and
    nothing past [n_tok][n_ff] written."""
    import torch
    import ingot_attn as ia

    rng = np.random.default_rng(n_tok * 3 + n_ff)
    x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
    raws = [gb.random_weights(t, n_ff, n_in, seed=n_in + 11 * i + 5) for i in range(2)]
    xd = _t(x, dev)
    wd = [_t(r.reshape(-1), dev) for r in raws]
    pad = 31
    out = _t(np.full(n_tok * n_ff + pad, np.nan, np.float32), dev)
    print(f"[proj] chunk gate/up silu {t} {n_tok}x{n_in}x{n_ff}", flush=True)
    ia.proj(wd, xd, [out], ia.proj_desc(t, n_in, [n_ff, n_ff], epilogue=ia.PROJ_SILU_GATE, n_tok=n_tok))
    g = _t(np.zeros(n_tok * n_ff, np.float32), dev)
    u = _t(np.zeros(n_tok * n_ff, np.float32), dev)
    ia.linear(wd[0], xd, g, ia.linear_desc(t, n_in, n_ff, n_tok, n_splits=1), use_workspace=False)
    ia.linear(wd[1], xd, u, ia.linear_desc(t, n_in, n_ff, n_tok, n_splits=1), use_workspace=False)
    got = out.cpu().numpy()
    if n_tok * n_ff % 4 == 0:  # ingot_silu_mul takes whole float4s
        ia.silu_mul(g, u, n_tok * n_ff)
        torch.cuda.synchronize()
        assert np.array_equal(got[: n_tok * n_ff], g.cpu().numpy()), f"{t}: != linear + linear + silu_mul"
    else:
        torch.cuda.synchronize()
        gh, uh = g.cpu().numpy().astype(np.float64), u.cpu().numpy().astype(np.float64)
        _close(got[: n_tok * n_ff], gh / (1.0 + np.exp(-gh)) * uh, f"{t}: vs linear + linear + silu")
    assert np.all(np.isnan(got[n_tok * n_ff:])), f"{t}: wrote past its rows"
    rows = sorted({0, 1, n_tok // 2, n_tok - 1})
    gg = oracle_mod.linear(t, raws[0], x[rows], n_in, n_ff, f16_path=True)
    uu = oracle_mod.linear(t, raws[1], x[rows], n_in, n_ff, f16_path=True)
    want = gg / (1.0 + np.exp(-gg)) * uu
    _close(got[: n_tok * n_ff].reshape(n_tok, n_ff)[rows], want, f"{t} chunk gate/up silu")
