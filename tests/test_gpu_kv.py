"""The GPU KV store (vireo_kv_*) against the reference's own stores
(src/kvstore_dense.c, src/kvstore_ooc.c, src/select/*, compiled into
oracle/_ref), fed the same appends and queries.

* Attention outputs within 2e-5 of their largest magnitude (fp32; the
  reference sums token by token, the GPU in parallel).
* Paging: with the same capacity, sinks, window and strategy the two stores
  make the same decisions, so every statistic (requests, hits, misses, bytes
  read and spilled, resident bytes) is equal after every query; TOPK selects
  the same blocks because the running mean keys and their scores are the
  reference's bits.
* The reference's invariant (src/kvstore.h:9-11): the out-of-core store with
  every block selected gives the dense store's result; here bit for bit, even
  with blocks spilled and paged back.
* Grouped-query attention in one launch equals the reference's per-head loop
  (src/gguf_run.c:233-235), statistics included.
"""
import numpy as np
import pytest
import torch

from vireo_amd import kv as KV

pytestmark = pytest.mark.gpu
TOL = 2e-5


@pytest.fixture(scope="module")
def ref():
    from oracle.oracle import Reference
    if not Reference.available():
        pytest.skip("oracle/_ref not built")
    return Reference()


def rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def drive(cuda, ref_kv, gpu_kv, n_layers, d, T, attend_every, seed, extra=None):
    """Append T tokens to every layer; every attend_every tokens query every
    layer on both stores and compare outputs and statistics."""
    rng = np.random.default_rng(seed)
    worst = 0.0
    out = torch.empty(d, dtype=torch.float32, device=cuda)
    for t in range(T):
        K = rng.standard_normal((n_layers, d)).astype(np.float32)
        V = rng.standard_normal((n_layers, d)).astype(np.float32)
        for l in range(n_layers):
            ref_kv.append(l, t, K[l], V[l])
        gpu_kv.append(0, t, torch.from_numpy(K).to(cuda), torch.from_numpy(V).to(cuda))
        if extra is not None:
            extra.append(0, t, torch.from_numpy(K).to(cuda), torch.from_numpy(V).to(cuda))
        if t % attend_every == attend_every - 1 or t == T - 1:
            for l in range(n_layers):
                q = rng.standard_normal(d).astype(np.float32)
                o_ref = ref_kv.attend(l, q)
                qg = torch.from_numpy(q).to(cuda)
                gpu_kv.attend(l, qg, out)
                worst = max(worst, rel(out.cpu().numpy(), o_ref))
                if extra is not None:
                    o2 = torch.empty_like(out)
                    extra.attend(l, qg, o2)
                    assert torch.equal(out, o2), (t, l)  # paged "all" == dense, bit for bit
                assert gpu_kv.stats() == ref_kv.stats(), (t, l, gpu_kv.stats(), ref_kv.stats())
    return worst


@pytest.mark.parametrize("d,G", [(64, 16), (128, 16), (256, 8), (128, 64)])
def test_dense_matches_reference(cuda, ref, d, G):
    from oracle.oracle import RefKV
    L, T = 3, 150
    r = RefKV(ref, L, d, G)
    g = KV.DeviceKV(L, d, G, dense=True)
    worst = drive(cuda, r, g, L, d, T, 13, seed=d + G)
    print(f"dense d={d} G={G}: max rel {worst:.2e}")
    assert worst <= TOL
    g.close()
    r.close()


@pytest.mark.parametrize("strategy", ["all", "recent", "topk"])
@pytest.mark.parametrize("tight", [False, True])
def test_paged_matches_reference(cuda, ref, strategy, tight):
    """Sinks of one block, a window of two, 4 layers of 200 tokens in blocks of
    16, queried every 10 tokens. Tight capacities: every layer's pinned blocks
    plus one layer's whole history (all), or plus the selection (recent, topk)."""
    from oracle.oracle import RefKV
    L, d, G, T, sink, window = 4, 128, 16, 200, 16, 32
    bb = 2 * G * d * 4
    nb = (T + G - 1) // G
    cap = 0
    if tight:
        cap = (4 * L + nb) * bb if strategy == "all" else (4 * L + 4) * bb
    code = {"all": KV.ALL, "recent": KV.RECENT, "topk": KV.TOPK}[strategy]
    r = RefKV(ref, L, d, G, sink, window, cap, strategy=strategy, budget=3)
    g = KV.DeviceKV(L, d, G, sink, window, cap, strategy=code, topk_budget=3)
    extra = KV.DeviceKV(L, d, G, dense=True) if strategy == "all" else None
    worst = drive(cuda, r, g, L, d, T, 10, seed=7, extra=extra)
    st = g.stats()
    print(f"paged {strategy} cap={cap}: max rel {worst:.2e}; {st}")
    assert worst <= TOL
    if tight:  # the pager was exercised: blocks leaving the window spill; the
        # selections of all / topk page some back (recent reads only pinned blocks)
        assert st["bytes_spilled"] > 0 and (st["misses"] > 0) == (strategy != "recent")
        assert st["resident_bytes"] <= cap
    for s in (g, r, extra):
        if s is not None:
            s.close()


@pytest.mark.parametrize("strategy", ["all", "topk"])
def test_gqa_matches_reference(cuda, ref, strategy):
    """8 query heads over 2 kv heads of each of 2 transformer layers (kv
    layers l * 2 + kv_head): one vireo_kv_attend_gqa per transformer layer
    against the reference's kv_attend per head."""
    from oracle.oracle import RefKV
    n_tl, n_kv, n_heads, d, G, T = 2, 2, 8, 128, 16, 120
    L = n_tl * n_kv
    code = {"all": KV.ALL, "topk": KV.TOPK}[strategy]
    r = RefKV(ref, L, d, G, 16, 32, 0, strategy=strategy, budget=2)
    g = KV.DeviceKV(L, d, G, 16, 32, 0, strategy=code, topk_budget=2)
    rng = np.random.default_rng(11)
    out = torch.empty((n_heads, d), dtype=torch.float32, device=cuda)
    worst = 0.0
    for t in range(T):
        K = rng.standard_normal((L, d)).astype(np.float32)
        V = rng.standard_normal((L, d)).astype(np.float32)
        for l in range(L):
            r.append(l, t, K[l], V[l])
        g.append(0, t, torch.from_numpy(K).to(cuda), torch.from_numpy(V).to(cuda))
        if t % 17 == 16 or t == T - 1:
            for tl in range(n_tl):
                q = rng.standard_normal((n_heads, d)).astype(np.float32)
                o_ref = np.stack([r.attend(tl * n_kv + h // (n_heads // n_kv), q[h]) for h in range(n_heads)])
                g.attend_gqa(tl * n_kv, n_heads, n_kv, torch.from_numpy(q).to(cuda), out)
                worst = max(worst, rel(out.cpu().numpy(), o_ref))
                assert g.stats() == r.stats()
    print(f"gqa {strategy}: max rel {worst:.2e}; {g.stats()}")
    assert worst <= TOL
    g.close()
    r.close()


@pytest.mark.parametrize("strategy", ["all", "topk"])
def test_gqa_long_context(cuda, ref, strategy):
    """A context long enough that the chunks' partials of one head number
    more than 64 (600 tokens in blocks of 4: 75 chunks of 2 blocks for the
    grouped kernel; top-k keeps 100 blocks for the per-head one), so the
    merge takes more than one pass over 64 chunks, against the reference's
    kv_attend per head."""
    from oracle.oracle import RefKV
    n_kv, n_heads, d, G, T = 1, 4, 64, 4, 600
    code = {"all": KV.ALL, "topk": KV.TOPK}[strategy]
    r = RefKV(ref, n_kv, d, G, 16, 32, 0, strategy=strategy, budget=100)
    g = KV.DeviceKV(n_kv, d, G, 16, 32, 0, strategy=code, topk_budget=100)
    rng = np.random.default_rng(12)
    out = torch.empty((n_heads, d), dtype=torch.float32, device=cuda)
    worst = 0.0
    for t in range(T):
        K = rng.standard_normal((n_kv, d)).astype(np.float32)
        V = rng.standard_normal((n_kv, d)).astype(np.float32)
        r.append(0, t, K[0], V[0])
        g.append(0, t, torch.from_numpy(K).to(cuda), torch.from_numpy(V).to(cuda))
        if t in (255, 520, T - 1):
            q = rng.standard_normal((n_heads, d)).astype(np.float32)
            o_ref = np.stack([r.attend(0, q[h]) for h in range(n_heads)])
            g.attend_gqa(0, n_heads, n_kv, torch.from_numpy(q).to(cuda), out)
            worst = max(worst, rel(out.cpu().numpy(), o_ref))
            assert g.stats() == r.stats()
    print(f"gqa long {strategy}: max rel {worst:.2e}; {g.stats()}")
    assert worst <= TOL
    g.close()
    r.close()


def test_empty_layer_attends_to_zero(cuda, ref):
    g = KV.DeviceKV(2, 64, 16, dense=True)
    q = torch.ones(64, dtype=torch.float32, device=cuda)
    out = torch.full((64,), 7.0, dtype=torch.float32, device=cuda)
    g.attend(1, q, out)
    assert torch.count_nonzero(out).item() == 0
    g.close()


@pytest.mark.parametrize("d,G", [(128, 32), (64, 16)])
def test_contiguous_store_equals_dense(cuda, d, G):
    """A contiguous store (blocks allocated up front) gives the dense store's
    grouped-query results bit for bit, driven by host positions and, in a third
    store, by device positions (vireo_kv_append_pos / vireo_kv_attend_gqa_pos,
    the calls a captured decode loop makes), across block boundaries."""
    n_tl, n_kv, n_heads, T = 2, 2, 8, 3 * G + 5
    L = n_tl * n_kv
    dense = KV.DeviceKV(L, d, G, dense=True)
    cont = KV.DeviceKV(L, d, G, dense=True, max_tokens=T)
    devp = KV.DeviceKV(L, d, G, dense=True, max_tokens=T)
    pos = torch.zeros(1, dtype=torch.int32, device=cuda)
    rng = np.random.default_rng(5)
    outs = [torch.empty((n_heads, d), dtype=torch.float32, device=cuda) for _ in range(3)]
    for t in range(T):
        K = torch.from_numpy(rng.standard_normal((L, d)).astype(np.float32)).to(cuda)
        V = torch.from_numpy(rng.standard_normal((L, d)).astype(np.float32)).to(cuda)
        dense.append(0, t, K, V)
        cont.append(0, t, K, V)
        pos.fill_(t)
        devp.append_pos(0, pos, K, V)
        if t % 7 == 6 or t == T - 1:
            for tl in range(n_tl):
                q = torch.from_numpy(rng.standard_normal((n_heads, d)).astype(np.float32)).to(cuda)
                dense.attend_gqa(tl * n_kv, n_heads, n_kv, q, outs[0])
                cont.attend_gqa(tl * n_kv, n_heads, n_kv, q, outs[1])
                devp.attend_gqa_pos(tl * n_kv, n_heads, n_kv, pos, q, outs[2])
                assert torch.equal(outs[0], outs[1]), (t, tl)
                assert torch.equal(outs[0], outs[2]), (t, tl)
    # a position past the store's tokens writes nothing
    pos.fill_(T)
    before = outs[2].clone()
    devp.append_pos(0, pos, K, V)
    pos.fill_(T - 1)
    devp.attend_gqa_pos(0, n_heads, n_kv, pos, q, outs[2])
    dense.attend_gqa(0, n_heads, n_kv, q, outs[0])
    assert torch.equal(outs[0], outs[2])
    del before
    for s in (dense, cont, devp):
        s.close()
