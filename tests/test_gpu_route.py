"""moe_route and moe_dispatch on the GPU: the chosen experts bit-exact with
the oracle (the reference picks by its own fp32 logits with a strict '>'
scan, src/gguf_run.c:189-191), including exactly tied experts, Zipf-biased
routers and the prefill path; dispatch against a stable sort."""
import numpy as np
import pytest
import torch

from vireo_amd import moe as M
from vireo_amd import workloads as W

pytestmark = pytest.mark.gpu

FALLBACK, NEAR_TIE = 1, 2


def oracle_route(oracle, shape, router, hb, bias=None):
    """Per-token (idx, w, probs) as moe_ffn computes them."""
    T = hb.shape[0]
    idx = np.empty((T, shape.k), np.int32)
    w = np.empty((T, shape.k), np.float32)
    probs = np.empty((T, shape.E), np.float32)
    for t in range(T):
        lg = oracle.matmul(W.F32, router, hb[t], shape.d, shape.E)
        if bias is not None:
            lg = (lg + bias).astype(np.float32)
        p = oracle.softmax(lg)
        probs[t] = p
        idx[t], w[t] = oracle.topk(p, shape.k, shape.renorm)
    return idx, w, probs


@pytest.mark.parametrize("name,T", [("qwen3-30b-a3b-q4_k_m", 1), ("qwen3-30b-a3b-q4_k_m", 37),
                                    ("olmoe-q8_0", 1), ("olmoe-q8_0", 16), ("qwen3-30b-a3b-q8_0", 64),
                                    ("olmoe-q4_k_m", 130)])
def test_route_matches_oracle(cuda, oracle, name, T):
    shape = W.SHAPES[name]
    m = M.DeviceMoE(shape, 1, seed=41)
    x, hb = W.host_hidden(shape.d, T, 41)
    idx, w, flags, probs = m.route(0, torch.from_numpy(hb).to(cuda), want_probs=True)
    oi, ow, op = oracle_route(oracle, shape, m.host_router(0), hb)
    np.testing.assert_array_equal(idx.cpu().numpy(), oi)
    np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(probs.cpu().numpy(), op, rtol=1e-5, atol=1e-8)
    fl = flags.cpu().numpy()
    assert not np.any(fl & NEAR_TIE)
    if T >= 64:  # prefill: exact sequential logits, never a fallback
        assert not np.any(fl & FALLBACK)
    m.close()


def test_route_exact_ties(cuda, oracle):
    """Experts with identical router rows tie exactly; the lowest index wins."""
    shape = W.SHAPES["olmoe-q8_0"]
    m = M.DeviceMoE(shape, 1, seed=43)
    r = m.routers[0]
    for a, b in ((5, 9), (9, 40), (12, 13), (60, 2)):
        r[b].copy_(r[a])
    x, hb = W.host_hidden(shape.d, 24, 43)
    router = m.host_router(0)
    # make the tied rows win for some tokens: align a token with expert 5's row
    hb[0] = router[5] / np.linalg.norm(router[5]) * np.sqrt(shape.d)
    hb[1] = router[12] / np.linalg.norm(router[12]) * np.sqrt(shape.d)
    for T in (1, 24, 64):
        h = np.concatenate([hb] * 3)[:T] if T > 24 else hb[:T]
        idx, w, flags, _ = m.route(0, torch.from_numpy(np.ascontiguousarray(h)).to(cuda))
        oi, ow, _ = oracle_route(oracle, shape, router, h)
        np.testing.assert_array_equal(idx.cpu().numpy(), oi)
        np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=1e-5)
        assert flags.cpu().numpy()[0] & NEAR_TIE  # a tie inside or at the edge of the top-k is reported
    got = idx.cpu().numpy()
    assert 5 in got[0] and 9 in got[0]
    m.close()


@pytest.mark.parametrize("T", [1, 5, 70])
def test_route_probability_ties(cuda, oracle, T):
    """Inputs scaled until most probabilities underflow to exactly zero: the
    reference ranks probabilities with the lowest id winning a tie, so the
    experts after the few nonzero ones are the lowest ids left, not the next
    largest logits (decode, routing and prefill paths)."""
    shape = W.SHAPES["qwen3-30b-a3b-q4_k_m"]
    m = M.DeviceMoE(shape, 1, seed=45)
    x, hb = W.host_hidden(shape.d, T, 45)
    hb *= np.float32(3.0e5)
    idx, w, flags, probs = m.route(0, torch.from_numpy(hb).to(cuda), want_probs=True)
    oi, ow, op = oracle_route(oracle, shape, m.host_router(0), hb)
    assert (ow == 0).any(axis=1).all()  # every token chooses zero-probability experts
    np.testing.assert_array_equal(idx.cpu().numpy(), oi)
    np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=1e-5, atol=1e-30)
    np.testing.assert_allclose(probs.cpu().numpy(), op, rtol=1e-5, atol=1e-30)
    assert np.all(flags.cpu().numpy() & NEAR_TIE)  # the zero ties are reported
    m.close()


def test_route_zipf_bias(cuda, oracle):
    shape = W.SHAPES["qwen3-30b-a3b-q8_0"]
    bias = W.zipf_bias(shape.E, 1.1, seed=3)
    m = M.DeviceMoE(shape, 1, seed=44, logit_bias=bias)
    x, hb = W.host_hidden(shape.d, 200, 44)
    idx, w, flags, _ = m.route(0, torch.from_numpy(hb).to(cuda))
    oi, ow, _ = oracle_route(oracle, shape, m.host_router(0), hb, bias)
    np.testing.assert_array_equal(idx.cpu().numpy(), oi)
    np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=1e-5)
    counts = np.bincount(oi.reshape(-1), minlength=shape.E)
    assert counts.max() > 4 * np.median(counts)  # the bias skews the load
    m.close()


@pytest.mark.parametrize("T,k,E,skew", [(1, 8, 128, 0), (7, 8, 64, 0), (2048, 8, 128, 0), (300, 1, 256, 0),
                                         (33, 4, 8, 0), (256, 8, 64, 0), (257, 8, 64, 0), (4096, 8, 128, 1.1),
                                         (1000, 3, 256, 1.1), (1001, 3, 256, 0), (16500, 8, 128, 1.1)])
def test_dispatch_is_a_stable_sort(cuda, T, k, E, skew):
    """One-workgroup form up to 2048 pairs (256 x 8 and 257 x 8 straddle the
    switch); above, one launch with a workgroup per expert when the pair
    count is a multiple of 4 and at most 131072 (2048 x 8, 4096 x 8,
    1000 x 3), else the two-kernel form (1001 x 3, 16500 x 8); skew draws
    experts with Zipf weights."""
    rng = np.random.default_rng(T * k + E)
    p = None
    if skew:
        p = 1.0 / np.arange(1, E + 1) ** skew
        p /= p.sum()
    idx = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    counts, offs, perm = M.dispatch(torch.from_numpy(idx).to(cuda), E)
    flat = idx.reshape(-1)
    np.testing.assert_array_equal(counts.cpu().numpy(), np.bincount(flat, minlength=E))
    np.testing.assert_array_equal(offs.cpu().numpy(), np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]))
    np.testing.assert_array_equal(perm.cpu().numpy(), np.argsort(flat, kind="stable"))


@pytest.mark.parametrize("case", ["random", "alternating", "range", "subnormal", "d1024"])
def test_router_logits_exact(cuda, oracle, lib, case):
    """vireo_router_logits is the reference's in-order fp32 chain bit for bit
    (the chain the routing kernels run for tokens they cannot certify). For
    d = 2048 a wave shares one chain, 32 steps per lane, and re-runs it until
    every lane starts from its neighbour's end, so the cases are the ones that
    make guessed starts wrong and keep them wrong: products of alternating sign
    that take the sum back across zero (a new binade) at every step,
    magnitudes over 36 decades, subnormal products and sums; d = 1024 takes
    one thread per chain."""
    import ctypes as C
    from vireo_amd import _lib
    rng = np.random.default_rng(71)
    d = 1024 if case == "d1024" else 2048
    E, T = 40, 5
    R = (rng.standard_normal((E, d)) * 0.05).astype(np.float32)
    hb = rng.standard_normal((T, d)).astype(np.float32)
    if case == "alternating":
        sign = np.where(np.arange(d) % 2 == 0, 1.0, -1.0).astype(np.float32)
        R = ((np.abs(R) + 0.5) * sign).astype(np.float32)
        hb = (np.abs(hb) * 1000.0 + 1.0).astype(np.float32)
    elif case == "range":
        hb = (hb * 10.0 ** rng.uniform(-18, 18, (T, d))).astype(np.float32)
    elif case == "subnormal":
        R = (R * 1e-20).astype(np.float32)
        hb = (hb * 1e-19).astype(np.float32)
    Rt, ht = torch.from_numpy(R).to(cuda), torch.from_numpy(hb).to(cuda)
    out = torch.empty((T, E), dtype=torch.float32, device=cuda)
    _lib.check(lib.vireo_router_logits(C.c_void_p(Rt.data_ptr()), C.c_void_p(ht.data_ptr()), d, E, T,
                                       C.c_void_p(out.data_ptr()), None), "vireo_router_logits")
    want = np.stack([oracle.matmul(W.F32, R, hb[t], d, E) for t in range(T)])
    got = out.cpu().numpy()
    if case == "subnormal":
        assert np.count_nonzero(np.abs(want) < 1.1754944e-38) > 0
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
