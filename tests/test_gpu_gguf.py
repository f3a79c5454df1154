"""MoE models read from GGUF files (vireo_gguf_moe_load) on the GPU, against
the oracle on the arrays that were written into the file.

* Layers: the loader binds every layer's router and expert tensors and
  registers expert e at offset + e * slice (src/gguf_run.c:320-333); each
  layer's moe_ffn_forward over a few tokens then matches the oracle's moe_ffn
  on the written router and expert bytes (routing exact, outputs within 2e-3
  of the layer's largest contribution). Shapes: Qwen3 Q4_K/Q6_K layers with
  16 experts (the one-token decode plan for single tokens) and d=256 layers
  of every expert type (the grouped plan). The metadata read back (top-k,
  widths, renormalisation rule by architecture, eps) is what was written.
* The store pages the experts from the file: after a layer's first call its
  resident bytes are the layer's expert bytes, read once.
* Stack: moe_stack_step on the file's ffn norms, output norm, LM head and
  token embedding (untied and tied) against the oracle's decode skeleton
  (src/gguf_run.c:216-254 with attention omitted), as in test_gpu_stack.
* A store smaller than a layer (the reference's laptop case): every call
  pages its routed experts in batches that fit; outputs match the oracle, and
  equal the fully resident model's bit for bit where both run the grouped
  kernels (more than one token); the pool never exceeds its capacity, the
  statistics equal the oracle's ExpertStore driven by the same tokens, and the
  stack decodes through it.
* Prefetch: the paged stack with and without reading the next layer's
  guessed experts ahead gives equal results bit for bit and equal statistics.
"""
import numpy as np
import pytest
import torch

from conftest import RefStoreReplay, expert_lists
from vireo_amd import gguf as G
from vireo_amd import workloads as W

pytestmark = pytest.mark.gpu
TOL = 2e-3

SHAPES = {
    "qwen3-16e": W.SHAPES["qwen3-30b-a3b-q4_k_m"].with_(name="qwen3-16e", E=16),
    "tiny-k": W.MoEShape("tiny-k", 256, 8, 2, 256, True, W.Q4_K, W.Q4_K, W.Q6_K),
    "tiny-q8": W.MoEShape("tiny-q8", 256, 8, 3, 256, False, W.Q8_0, W.Q8_0, W.Q8_0),
}


def check(name, x, xg, xo, idx_g, idx_o):
    np.testing.assert_array_equal(idx_g, idx_o)
    dg, do = xg - x, xo - x
    rel = np.abs(dg - do).max() / np.abs(do).max()
    print(f"{name}: max rel {rel:.2e}")
    assert rel <= TOL


@pytest.mark.parametrize("name", list(SHAPES))
def test_gguf_layers_match_oracle(cuda, oracle, tmp_path, name):
    shape, L = SHAPES[name], 2
    path = tmp_path / f"{name}.gguf"
    arr = G.write_moe_gguf(str(path), shape, L, seed=29)
    m = G.GGUFModel(path, load_head=False)
    assert (m.arch, m.n_layers, m.d, m.E, m.k, m.fe, m.renorm) == (G.moe_arch(shape), L, shape.d, shape.E,
                                                                    shape.k, shape.fe, shape.renorm)
    assert m.eps == np.float32(W.EPS)
    gs, us, ds = shape.slice_bytes()
    replay = RefStoreReplay(oracle, shape, L, 0)
    for layer in range(L):
        Gl, Ul, Dl = expert_lists(shape, *arr["experts"][layer])
        for T in (1, 5):
            x, hb = W.host_hidden(shape.d, T, seed=layer * 7 + T)
            xg, hg = torch.from_numpy(x).to(cuda), torch.from_numpy(hb).to(cuda)
            idx, _ = m.forward(layer, xg, hg, return_routing=True)
            xo, io, _, _ = oracle.moe_ffn(shape, arr["routers"][layer], Gl, Ul, Dl, x, hb)
            check(f"{name} layer {layer} T={T}", x, xg.cpu().numpy(), xo, idx.cpu().numpy(), io)
            replay.route(layer, io)
        # the pool holds whole layers, each read from the file once (and the
        # decode batch's tiled copies of the Q4_K_M layers)
        hbm = m.hbm_stats()
        assert hbm["resident_bytes"] == (layer + 1) * shape.E * (gs + us + ds) + m.packed_bytes()
        assert hbm["bytes_read"] == (layer + 1) * shape.E * (gs + us + ds)
        # the statistics are the reference's for the same tokens
        assert m.stats() == replay.stats()
    replay.close()
    m.close()


def oracle_stack(oracle, shape, arr, L, vocab):
    d = shape.d
    rb = W.row_bytes(W.Q8_0, d)
    emb, head = arr["token_embd"], arr["output"]
    layers = [expert_lists(shape, *arr["experts"][l]) for l in range(L)]

    def step(tok):
        x = oracle.dequant_row(W.Q8_0, emb[tok * rb:(tok + 1) * rb], d)
        for l in range(L):
            xb = oracle.rmsnorm(x, arr["ffn_norm"][l], W.EPS)
            x = oracle.moe_ffn(shape, arr["routers"][l], *layers[l], x, xb)[0][0]
        logits = oracle.matmul(W.Q8_0, head, oracle.rmsnorm(x, arr["out_norm"], W.EPS), d, vocab)
        return x, logits, oracle.argmax(logits)
    return step


@pytest.mark.parametrize("name,untied,cap_experts", [("tiny-k", True, 0), ("tiny-k", False, 0), ("qwen3-16e", True, 0),
                                                     ("qwen3-16e", True, 5)])
def test_gguf_stack_matches_oracle(cuda, oracle, tmp_path, name, untied, cap_experts):
    """qwen3-16e runs the one-token decode plan, whose router launch applies
    the file's RMSNorm weights itself, or, with a store of 5 experts, the
    paged plan; tiny-k the grouped plan."""
    shape, L, vocab = SHAPES[name], 3, 700
    path = tmp_path / "stack.gguf"
    arr = G.write_moe_gguf(str(path), shape, L, seed=37, vocab=vocab, untied=untied)
    m = G.GGUFModel(path, expert_capacity=cap_experts * shape.expert_bytes())
    assert m.vocab == vocab
    ref = oracle_stack(oracle, shape, arr, L, vocab)
    x = torch.empty(shape.d, dtype=torch.float32, device=cuda)
    xb = torch.empty_like(x)
    logits = torch.empty(vocab, dtype=torch.float32, device=cuda)
    token = torch.empty(1, dtype=torch.int32, device=cuda)
    for i, tok in enumerate((5, vocab - 1, vocab // 2, 0)):
        token.fill_(tok)
        m.step(token, x, xb, logits)
        xo, lo, to = ref(tok)
        xg, lg, tg = x.cpu().numpy(), logits.cpu().numpy(), int(token.cpu()[0])
        rx = np.abs(xg - xo).max() / np.abs(xo).max()
        rl = np.abs(lg - lo).max() / np.abs(lo).max()
        print(f"{name} untied={untied} step {i}: token {tok} -> {tg} (oracle {to}); x {rx:.2e}, logits {rl:.2e}")
        assert rx <= TOL and rl <= TOL
        top2 = np.sort(lo)[-2:]
        if top2[1] - top2[0] > TOL * np.abs(lo).max():
            assert tg == to
    m.close()


@pytest.mark.parametrize("name,cap_experts,T,L", [("tiny-k", 3, 5, 2), ("tiny-q8", 1, 3, 2), ("qwen3-16e", 4, 1, 2),
                                                 ("qwen3-16e", 5, 6, 2), ("qwen3-16e", 24, 1, 3),
                                                 ("tiny-k", 12, 4, 3)])
def test_gguf_paged_store(cuda, oracle, tmp_path, name, cap_experts, T, L):
    """Stores smaller than the model (down to one expert, and about one and
    a half layers of a 3-layer model): the pool stays within its capacity,
    outputs match the oracle, and the statistics are the reference's for the
    same tokens."""
    shape = SHAPES[name]
    path = tmp_path / f"{name}.gguf"
    arr = G.write_moe_gguf(str(path), shape, L, seed=41)
    cap = cap_experts * shape.expert_bytes()
    paged = G.GGUFModel(path, expert_capacity=cap, load_head=False)
    full = G.GGUFModel(path, load_head=False)
    replay = RefStoreReplay(oracle, shape, L, cap)
    for call in range(3 * L):
        layer = call % L
        Gl, Ul, Dl = expert_lists(shape, *arr["experts"][layer])
        x, hb = W.host_hidden(shape.d, T, seed=100 + call)
        xp, hp = torch.from_numpy(x).to(cuda), torch.from_numpy(hb).to(cuda)
        xf = xp.clone()
        idx, _ = paged.forward(layer, xp, hp, return_routing=True)
        full.forward(layer, xf, hp)
        xo, io, _, _ = oracle.moe_ffn(shape, arr["routers"][layer], Gl, Ul, Dl, x, hb)
        check(f"{name} paged call {call} layer {layer}", x, xp.cpu().numpy(), xo, idx.cpu().numpy(), io)
        if T > 1:  # both on the grouped kernels: the same rows, the same combine
            assert torch.equal(xp, xf)
        replay.route(layer, io)
        hbm = paged.hbm_stats()
        assert hbm["resident_bytes"] <= cap, hbm
        assert paged.stats() == replay.stats()
    print(f"{name} cap {cap_experts} experts: {paged.stats()}; pool {paged.hbm_stats()}")
    replay.close()
    paged.close()
    full.close()


@pytest.mark.parametrize("name,cap_experts,L", [("qwen3-16e", 12, 4), ("tiny-k", 6, 4)])
def test_gguf_prefetch_changes_no_result(cuda, oracle, tmp_path, name, cap_experts, L):
    """Paged decode through the stack with the next-layer guess on and off:
    every step's state, logits and token are equal bit for bit (the guess
    changes what the pool holds, not the batches or kernels), the reference's
    statistics are equal, the pool stays within its capacity, and guessed
    experts are read ahead and then looked up (the residual stream moves
    little between layers, so the next router's choice on this layer's input
    is often right)."""
    shape, vocab = SHAPES[name], 300
    path = tmp_path / "pf.gguf"
    G.write_moe_gguf(str(path), shape, L, seed=53, vocab=vocab)
    cap = cap_experts * shape.expert_bytes()
    runs = {}
    for on in (True, False):
        m = G.GGUFModel(path, expert_capacity=cap)
        m.set_prefetch(on)
        x = torch.empty(shape.d, dtype=torch.float32, device=cuda)
        xb = torch.empty_like(x)
        logits = torch.empty(vocab, dtype=torch.float32, device=cuda)
        token = torch.full((1,), 7, dtype=torch.int32, device=cuda)
        stream = torch.cuda.Stream()
        seen = []
        for _ in range(6):
            m.step(token, x, xb, logits, stream=stream)
            torch.cuda.synchronize()
            seen.append((x.cpu().clone(), logits.cpu().clone(), int(token.cpu()[0])))
            assert m.hbm_stats()["resident_bytes"] <= cap
        runs[on] = (seen, m.stats(), m.prefetch_stats())
        m.close()
    (a, sa, pa), (b, sb, pb) = runs[True], runs[False]
    for i, ((xa, la, ta), (xb_, lb, tb)) in enumerate(zip(a, b)):
        assert torch.equal(xa, xb_) and torch.equal(la, lb) and ta == tb, f"step {i}"
    assert sa == sb
    print(f"{name}: prefetch {pa}; off {pb}")
    assert pb == {"issued": 0, "used": 0, "bytes": 0}
    assert pa["issued"] > 0 and 0 < pa["used"] <= pa["issued"]
    assert pa["bytes"] == pa["issued"] * shape.expert_bytes()
