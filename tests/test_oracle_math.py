"""Pins of the oracle by what the mathematics fixes, independent of its code:
IEEE half conversion over every bit pattern, the GGUF block layouts decoded
by a separate numpy decoder, error bounds of the dot products, closed forms
of softmax/RMSNorm, brute-force top-k with lowest-index tie-break, and a
float64 restatement of the whole MoE layer built from those pieces.
"""
import numpy as np
import pytest

import qformats as Q
from conftest import expert_lists
from vireo_amd import workloads as W

U24 = 2.0 ** -24


def test_f16_all_bit_patterns(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _random_blocks(typ, rows, n, rng):
    """Uniform random bytes with the f16 scale fields replaced by finite values,
    so every quant bit pattern is exercised."""
    be, bb = Q.BLOCK[typ]
    raw = rng.integers(0, 256, size=(rows * n // be, bb), dtype=np.uint8)
    fields = {Q.Q8_0: [0], Q.Q5_0: [0], Q.Q4_K: [0, 2], Q.Q6_K: [208]}[typ]
    for off in fields:
        raw[:, off:off + 2] = (rng.standard_normal(raw.shape[0]) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return raw.reshape(-1)


@pytest.mark.parametrize("typ,n", [(Q.Q8_0, 256), (Q.Q5_0, 256), (Q.Q4_K, 512), (Q.Q6_K, 512)])
def test_dequant_matches_format_decoder(oracle, typ, n):
    rng = np.random.default_rng(typ)
    rows = 24
    raw = _random_blocks(typ, rows, n, rng)
    want = Q.decode(typ, raw, n)
    rb = raw.size // rows
    got = np.stack([oracle.dequant_row(typ, raw[i * rb:(i + 1) * rb], n) for i in range(rows)])
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("typ,n,d", [(Q.Q8_0, 2048, 64), (Q.Q4_K, 2048, 64), (Q.Q6_K, 768, 64), (Q.Q5_0, 512, 32),
                                     (Q.F16, 300, 16), (Q.F32, 2048, 128)])
def test_matmul_error_bound(oracle, typ, n, d):
    """|y - W x| <= (n+2) u sum|w x| for any summation order of fp32 products."""
    rng = np.random.default_rng(100 + typ)
    if typ == Q.F32:
        w = rng.standard_normal(n * d).astype(np.float32) * 0.02
        wd = w.reshape(d, n).astype(np.float64)
    elif typ == Q.F16:
        w = (rng.standard_normal(n * d) * 0.1).astype(np.float16).view(np.uint8)
        wd = Q.decode(typ, w, n).astype(np.float64)
    else:
        w = _random_blocks(typ, d, n, rng)
        wd = Q.decode(typ, w, n).astype(np.float64)
    x = rng.standard_normal(n).astype(np.float32)
    y = oracle.matmul(typ, w, x, n, d).astype(np.float64)
    exact = wd @ x.astype(np.float64)
    bound = (n + 2) * U24 * (np.abs(wd) @ np.abs(x.astype(np.float64))) + 1e-30
    assert np.all(np.abs(y - exact) <= bound)
    # the bound is tight enough that a dropped 32-element block fails it on most rows
    assert np.mean(np.abs((wd[:, 32:] @ x[32:]) - exact) > bound) > 0.5


def test_softmax_closed_form(oracle):
    rng = np.random.default_rng(1)
    for n in (1, 8, 64, 128, 256):
        v = (rng.standard_normal(n) * 3).astype(np.float32)
        p = oracle.softmax(v).astype(np.float64)
        e = np.exp(v.astype(np.float64) - v.max())
        np.testing.assert_allclose(p, e / e.sum(), rtol=2e-6, atol=1e-12)
        assert abs(p.sum() - 1.0) < 1e-5


def test_rmsnorm_closed_form(oracle):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(2048).astype(np.float32)
    w = rng.standard_normal(2048).astype(np.float32)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean() + 1e-6) * w
    np.testing.assert_allclose(oracle.rmsnorm(x, w, 1e-6), want, rtol=2e-5, atol=1e-7)


def _topk_brute(p, k, renorm):
    order = sorted(range(len(p)), key=lambda e: (-float(p[e]), e))[:min(k, 64)]
    w = np.array([p[e] for e in order], np.float32)
    if renorm and w.sum() > 0:
        w = (w.astype(np.float64) / w.astype(np.float64).sum())
    return np.array(order, np.int32), w


@pytest.mark.parametrize("renorm", [False, True])
def test_topk_brute_force_with_ties(oracle, renorm):
    rng = np.random.default_rng(3)
    cases = [rng.random(64).astype(np.float32),
             np.full(16, 0.0625, np.float32),                         # all tied: lowest indices win
             np.repeat(rng.random(8).astype(np.float32), 4),          # pairs of ties
             np.array([0.1, 0.3, 0.3, 0.2, 0.3, 0.1], np.float32)]
    for p in cases:
        for k in (1, 2, 4, min(8, len(p)), len(p)):
            idx, w = oracle.topk(p, k, renorm)
            bi, bw = _topk_brute(p, k, renorm)
            np.testing.assert_array_equal(idx, bi)
            np.testing.assert_allclose(w, bw, rtol=1e-6)


def test_argmax_first_occurrence(oracle):
    assert oracle.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert oracle.argmax(np.array([-5, -1, -7], np.float32)) == 1
    v = np.random.default_rng(4).standard_normal(151936).astype(np.float32)
    assert oracle.argmax(v) == int(np.argmax(v))


def _moe64(shape, router, G, U, D, x, hb, bias=None):
    """float64 MoE layer from the format decoder: routing by exact logits,
    SwiGLU experts, weighted sum, residual. Returns (x_out, idx, margin)."""
    T = x.shape[0]
    logits = hb.astype(np.float64) @ router.astype(np.float64).T
    if bias is not None:
        logits = logits + bias
    out = x.astype(np.float64).copy()
    idxs, margins = [], []
    k = shape.k
    for t in range(T):
        p = np.exp(logits[t] - logits[t].max())
        p /= p.sum()
        order = np.argsort(-p, kind="stable")
        sel = order[:k]
        margins.append(p[order[k - 1]] - p[order[k]] if k < len(p) else 1.0)
        w = p[sel]
        if shape.renorm:
            w = w / w.sum()
        for j, e in enumerate(sel):
            if G[e] is None:
                continue
            g = Q.decode(shape.gate_type, G[e], shape.d).astype(np.float64) @ hb[t]
            u = Q.decode(shape.up_type, U[e], shape.d).astype(np.float64) @ hb[t]
            h = g / (1 + np.exp(-g)) * u
            out[t] += w[j] * (Q.decode(shape.down_type, D[e], shape.fe).astype(np.float64) @ h)
        idxs.append(sel)
    return out, np.array(idxs), np.array(margins)


@pytest.mark.parametrize("shape", [
    W.MoEShape("tiny-q4_k_m", 256, 16, 4, 256, True, W.Q4_K, W.Q4_K, W.Q6_K),
    W.MoEShape("tiny-q8_0", 256, 8, 2, 128, False, W.Q8_0, W.Q8_0, W.Q8_0),
    W.MoEShape("tiny-q5_0", 128, 8, 3, 64, False, W.Q5_0, W.Q5_0, W.Q8_0),
])
def test_moe_ffn_float64(oracle, shape):
    """The oracle's MoE layer against a float64 restatement assembled from the
    independent decoder; an unregistered expert is skipped as the reference's
    moe_ffn does when expert_store_lookup fails."""
    seed = 77
    router = W.host_router(shape, 0, seed)
    G, U, D = expert_lists(shape, *W.host_layer(shape, 0, seed))
    x, hb = W.host_hidden(shape.d, 6, seed)
    bias = (np.random.default_rng(5).standard_normal(shape.E) * 0.5).astype(np.float32)
    for b in (None, bias):
        xo, idx, w, probs = oracle.moe_ffn(shape, router, G, U, D, x, hb, bias=b)
        want, widx, margin = _moe64(shape, router, G, U, D, x, hb, None if b is None else b.astype(np.float64))
        assert np.all(margin > 1e-6)
        np.testing.assert_array_equal(idx, widx)
        delta, wdelta = xo - x, want - x
        assert np.abs(delta - wdelta).max() <= 1e-4 * np.abs(wdelta).max()
    # an unregistered expert contributes nothing
    G2 = list(G)
    U2, D2 = list(U), list(D)
    drop = int(idx[0, 0])
    G2[drop] = U2[drop] = D2[drop] = None
    xo2, idx2, _, _ = oracle.moe_ffn(shape, router, G2, U2, D2, x, hb, bias=bias)
    want2, _, _ = _moe64(shape, router, G2, U2, D2, x, hb, bias.astype(np.float64))
    assert np.abs((xo2 - x) - (want2 - x)).max() <= 1e-4 * np.abs(want2 - x).max()
    assert not np.allclose(xo2, xo)
