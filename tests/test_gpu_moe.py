"""moe_ffn_forward on the GPU against the oracle (the reference's moe_ffn,
src/gguf_run.c:185-214, restated) and against the golden vectors the
reference itself wrote, on both execution plans.

Bar: the routed experts bit-exact; the layer's contribution (x_out - x)
within 2e-3 of its largest magnitude (1e-2 where groups run as bf16
matrix-core GEMMs); the mean absolute error is printed.
"""
import numpy as np
import pytest
import torch

from conftest import expert_lists, golden
from vireo_amd import _lib
from vireo_amd import moe as M
from vireo_amd import workloads as W

pytestmark = pytest.mark.gpu
TOL = 2e-3
TOL_BF16 = 1e-2  # calls of >= 64 tokens: every group as bf16 GEMMs


@pytest.fixture
def path(request):
    lib = _lib.load()
    yield lambda p: lib.vireo_hip_set_path(p)
    lib.vireo_hip_set_path(0)


def oracle_layer(oracle, m, layer, x, hb, tokens=None):
    shape = m.shape
    G, U, D = expert_lists(shape, *m.host_layer(layer))
    for (l, e) in getattr(m, "_unregistered", ()):
        if l == layer:
            G[e] = U[e] = D[e] = None
    bias = m.bias.cpu().numpy() if m.bias is not None else None
    sel = slice(None) if tokens is None else tokens
    return oracle.moe_ffn(shape, m.host_router(layer), G, U, D, x[sel], hb[sel], bias=bias)


def check(name, x, xg, xo, idx_g, idx_o, tol=TOL):
    np.testing.assert_array_equal(idx_g, idx_o)
    dg, do = xg - x, xo - x
    err = np.abs(dg - do)
    rel = err.max() / np.abs(do).max()
    print(f"{name}: max rel {rel:.2e}  mean abs {err.mean():.2e}")
    assert rel <= tol


CONFIGS = [("olmoe-q8_0", 1), ("olmoe-q4_k_m", 1), ("olmoe-q4_k_m", 4), ("olmoe-q4_k_m", 16),
           ("qwen3-30b-a3b-q4_k_m", 1), ("qwen3-30b-a3b-q4_k_m", 32), ("qwen3-30b-a3b-q8_0", 1),
           ("qwen3-30b-a3b-q8_0", 80)]


@pytest.mark.parametrize("name,T", CONFIGS)
@pytest.mark.parametrize("plan", [0, 2, 3, 5])
def test_moe_ffn_matches_oracle(cuda, oracle, path, name, T, plan):
    if plan in (3, 5) and T > 1:
        pytest.skip("plans 3 and 5 (fused experts kernel, whole-layer kernel) are one-token decode plans")
    path(plan)
    shape = W.SHAPES[name]
    m = M.DeviceMoE(shape, 1, seed=51)
    x, hb = W.host_hidden(shape.d, T, 51)
    xt = torch.from_numpy(x).to(cuda)
    idx, w = m.forward(0, xt, torch.from_numpy(hb).to(cuda), return_routing=True)
    xo, io, wo, _ = oracle_layer(oracle, m, 0, x, hb)
    # calls of >= 64 tokens run every group as bf16 matrix-core GEMMs under plans 0 and 2
    tol = TOL_BF16 if T >= 64 and plan in (0, 2) else TOL
    check(f"{name} T={T} plan={plan}", x, xt.cpu().numpy(), xo, idx.cpu().numpy(), io, tol=tol)
    np.testing.assert_allclose(w.cpu().numpy(), wo, rtol=1e-5)
    m.close()


WIDE_TYPES = {"q6k-q6k-q8": (W.Q6_K, W.Q6_K, W.Q8_0), "q8-q8-q4k": (W.Q8_0, W.Q8_0, W.Q4_K),
              "q4k-q4k-q6k": (W.Q4_K, W.Q4_K, W.Q6_K)}


# expert types beyond the MoE models' own, which the reference's moe_ffn hands
# to gguf_matmul like any other (src/gguf_run.c:202-208; Q5_0 dequant-then-dot,
# F16 and F32 direct, src/gguf_compute.c:68-82, 183-213): the grouped fp32 kernels
OTHER_TYPES = {"q5_0-q5_0-q5_0": (W.Q5_0, W.Q5_0, W.Q5_0), "f16-f16-f16": (W.F16, W.F16, W.F16),
               "f32-f32-f32": (W.F32, W.F32, W.F32), "q5_0-q5_0-f16": (W.Q5_0, W.Q5_0, W.F16),
               "f16-f16-q6k": (W.F16, W.F16, W.Q6_K), "q4k-q4k-f32": (W.Q4_K, W.Q4_K, W.F32)}


@pytest.mark.parametrize("types", list(OTHER_TYPES))
@pytest.mark.parametrize("T", [1, 24, 80])
def test_other_expert_types(cuda, oracle, types, T):
    """Q5_0, F16 and F32 experts (alone and mixed with the K-quants) at one
    token, a decode batch and a call of more than 64 tokens, against the
    oracle; every call takes the grouped fp32 kernels."""
    shape = W.MoEShape("other-" + types, 2048, 16, 4, 512, True, *OTHER_TYPES[types])
    m = M.DeviceMoE(shape, 1, seed=57)
    x, hb = W.host_hidden(shape.d, T, 57)
    xt = torch.from_numpy(x).to(cuda)
    idx, w = m.forward(0, xt, torch.from_numpy(hb).to(cuda), return_routing=True)
    xo, io, wo, _ = oracle_layer(oracle, m, 0, x, hb)
    check(f"{shape.name} T={T}", x, xt.cpu().numpy(), xo, idx.cpu().numpy(), io)
    np.testing.assert_allclose(w.cpu().numpy(), wo, rtol=1e-5)
    m.close()


@pytest.mark.parametrize("types", list(WIDE_TYPES))
@pytest.mark.parametrize("T", [3, 24])
def test_decode_batch_every_type(cuda, oracle, types, T):
    """Calls of a few tokens on d = 2048 layers of every gate/up and down type;
    with 24 tokens over 16 experts most groups hold more tokens than one pass of
    the decode-batch kernels takes, and a few hold one."""
    shape = W.MoEShape("wide-" + types, 2048, 16, 4, 512, True, *WIDE_TYPES[types])
    m = M.DeviceMoE(shape, 1, seed=53)
    x, hb = W.host_hidden(shape.d, T, 53)
    xt = torch.from_numpy(x).to(cuda)
    idx, w = m.forward(0, xt, torch.from_numpy(hb).to(cuda), return_routing=True)
    xo, io, wo, _ = oracle_layer(oracle, m, 0, x, hb)
    check(f"{shape.name} T={T}", x, xt.cpu().numpy(), xo, idx.cpu().numpy(), io)
    counts = np.bincount(io.reshape(-1), minlength=shape.E)
    if T == 24:
        assert counts.max() > 4 and (counts == 1).any() or counts.max() > 4
    m.close()


@pytest.mark.parametrize("name", ["qwen3-30b-a3b-q4_k_m", "olmoe-q4_k_m", "olmoe-q8_0"])
@pytest.mark.parametrize("T", [2, 3, 5, 8])
def test_decode_batch_equals_one_token_calls(cuda, oracle, path, name, T):
    """Calls of 2 to 8 tokens on the decode plan (plan 1) give every token the
    bits of a one-token call - its routed experts, their weights and its x -
    also for a token whose order the fp64 bounds leave open (its inputs scaled
    so that most probabilities underflow: ranked again on exact logits) and,
    on the OLMoE Q4_K_M layer, with two experts unregistered; and they match
    the oracle."""
    path(1)
    shape = W.SHAPES[name]
    unreg = {(0, 3), (0, 17)} if name == "olmoe-q4_k_m" else set()
    m = M.DeviceMoE(shape, 1, seed=71 + T, unregistered=unreg)
    x, hb = W.host_hidden(shape.d, T, 71 + T)
    hb[T // 2] *= np.float32(3.0e5)
    xt = torch.from_numpy(x).to(cuda)
    hbt = torch.from_numpy(hb).to(cuda)
    idx, w = m.forward(0, xt, hbt, return_routing=True)
    xb, ib, wb = xt.cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy()
    for t in range(T):
        x1 = torch.from_numpy(x[t:t + 1].copy()).to(cuda)
        i1, w1 = m.forward(0, x1, hbt[t:t + 1], return_routing=True)
        np.testing.assert_array_equal(ib[t:t + 1], i1.cpu().numpy())
        np.testing.assert_array_equal(wb[t:t + 1].view(np.uint32), w1.cpu().numpy().view(np.uint32))
        np.testing.assert_array_equal(xb[t:t + 1].view(np.uint32), x1.cpu().numpy().view(np.uint32))
    xo, io, wo, _ = oracle_layer(oracle, m, 0, x, hb)
    check(f"decode batch {name} T={T}", x, xb, xo, ib, io)
    np.testing.assert_allclose(wb, wo, rtol=1e-5, atol=1e-30)
    m.close()


# shapes beyond the models': more than 128 experts (four router parts per
# lane), a count that is no multiple of 64 with unregistered experts, top-16
# and top-1, a wider expert; every one at up to the 64 (token, expert) pairs
BATCH_SHAPES = [
    (W.MoEShape("batch-e256", 2048, 256, 8, 512, True, W.Q4_K, W.Q4_K, W.Q6_K), 8, ()),
    (W.MoEShape("batch-e40-k4", 2048, 40, 4, 768, False, W.Q8_0, W.Q8_0, W.Q8_0), 8, ((0, 5), (0, 39))),
    (W.MoEShape("batch-k16", 2048, 128, 16, 768, True, W.Q4_K, W.Q4_K, W.Q6_K), 4, ()),
    (W.MoEShape("batch-k1", 2048, 16, 1, 1024, False, W.Q6_K, W.Q6_K, W.Q8_0), 7, ()),
    (W.MoEShape("batch-fe1536", 2048, 64, 8, 1536, False, W.Q4_K, W.Q4_K, W.Q6_K), 8, ()),
]


@pytest.mark.parametrize("shape,T,unreg", BATCH_SHAPES, ids=[s[0].name for s in BATCH_SHAPES])
def test_decode_batch_shapes(cuda, oracle, path, shape, T, unreg):
    """The decode plan for a batch (plan 1) on shapes beyond the models':
    every token gets the bits of a one-token call, one of them through the
    exact ranking, and the batch matches the oracle."""
    path(1)
    m = M.DeviceMoE(shape, 1, seed=81 + T, unregistered=set(unreg))
    x, hb = W.host_hidden(shape.d, T, 81 + T)
    hb[T // 2] *= np.float32(3.0e5)
    xt = torch.from_numpy(x).to(cuda)
    hbt = torch.from_numpy(hb).to(cuda)
    idx, w = m.forward(0, xt, hbt, return_routing=True)
    xb, ib, wb = xt.cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy()
    for t in range(T):
        x1 = torch.from_numpy(x[t:t + 1].copy()).to(cuda)
        i1, w1 = m.forward(0, x1, hbt[t:t + 1], return_routing=True)
        np.testing.assert_array_equal(ib[t:t + 1], i1.cpu().numpy())
        np.testing.assert_array_equal(wb[t:t + 1].view(np.uint32), w1.cpu().numpy().view(np.uint32))
        np.testing.assert_array_equal(xb[t:t + 1].view(np.uint32), x1.cpu().numpy().view(np.uint32))
    xo, io, wo, _ = oracle_layer(oracle, m, 0, x, hb)
    check(f"decode batch {shape.name} T={T}", x, xb, xo, ib, io)
    m.close()


def test_decode_batch_falls_back_past_its_lds(cuda, oracle, path):
    """A batch whose outputs would not fit the gate/up kernel's LDS (8 tokens,
    64 experts of width 2048) takes the grouped plan, also under plan 1."""
    path(1)
    shape = W.MoEShape("batch-fe2048", 2048, 64, 8, 2048, False, W.Q8_0, W.Q8_0, W.Q8_0)
    m = M.DeviceMoE(shape, 1, seed=89)
    x, hb = W.host_hidden(shape.d, 8, 89)
    xt = torch.from_numpy(x).to(cuda)
    idx, w = m.forward(0, xt, torch.from_numpy(hb).to(cuda), return_routing=True)
    xo, io, wo, _ = oracle_layer(oracle, m, 0, x, hb)
    check(f"decode batch fallback {shape.name}", x, xt.cpu().numpy(), xo, idx.cpu().numpy(), io)
    m.close()


@pytest.mark.parametrize("plan", [0, 1, 3, 5])
def test_decode_probability_ties(cuda, oracle, path, plan):
    """A token whose inputs are so large that all but a few probabilities
    underflow to zero: every one-token plan chooses as the reference does (the
    lowest ids among the zero-probability experts)."""
    path(plan)
    shape = W.SHAPES["qwen3-30b-a3b-q4_k_m"]
    m = M.DeviceMoE(shape, 1, seed=58)
    x, hb = W.host_hidden(shape.d, 1, 58)
    hb *= np.float32(3.0e5)
    xt = torch.from_numpy(x).to(cuda)
    idx, w = m.forward(0, xt, torch.from_numpy(hb).to(cuda), return_routing=True)
    xo, io, wo, _ = oracle_layer(oracle, m, 0, x, hb)
    assert (wo == 0).any()
    check(f"probability ties plan={plan}", x, xt.cpu().numpy(), xo, idx.cpu().numpy(), io)
    np.testing.assert_allclose(w.cpu().numpy(), wo, rtol=1e-5, atol=1e-30)
    m.close()


@pytest.mark.parametrize("T", [1, 2, 3, 8, 40])
@pytest.mark.parametrize("plan", [0, 2, 4])
def test_decode_batch_matrix_cores(cuda, oracle, path, T, plan):
    """Q4_K_M calls of 3 to 63 tokens run on the matrix cores under plan 2
    (under plan 0 from 5 tokens; 2 to 4 take the decode plan), smaller calls
    and plan 4 on the fp32 decode-batch kernels (T=2 and T=3 sit on either
    side of the switch under plan 2). With 40 tokens over 8 experts (top 4)
    every group holds more than one 16-token tile. Token 0's
    inputs are scaled past the fp16 range (their split takes a power of two
    per token) and token 1's far below it."""
    path(plan)
    shape = W.MoEShape("mdec-8e", 2048, 8, 4, 768, True, W.Q4_K, W.Q4_K, W.Q6_K)
    m = M.DeviceMoE(shape, 1, seed=57)
    x, hb = W.host_hidden(shape.d, T, 57)
    hb[0] *= 3.0e5
    if T > 1:  # a contribution of about 1e-12: the residual is zeroed so that it shows in x
        hb[1] *= 1.0e-6
        x[1] = 0.0
    xt = torch.from_numpy(x).to(cuda)
    idx, w = m.forward(0, xt, torch.from_numpy(hb).to(cuda), return_routing=True)
    xo, io, wo, _ = oracle_layer(oracle, m, 0, x, hb)
    np.testing.assert_array_equal(idx.cpu().numpy(), io)
    xg = xt.cpu().numpy()
    for t in range(T):  # per token: token 0's contribution is 10^11 times token 1's
        check(f"mdec T={T} plan={plan} token {t}", x[t:t + 1], xg[t:t + 1], xo[t:t + 1], io[t:t + 1], io[t:t + 1])
    if T == 40:  # most groups span two token tiles
        assert (np.bincount(io.reshape(-1), minlength=shape.E) > 16).sum() >= 4
    m.close()


@pytest.mark.parametrize("T", [8, 40])
def test_decode_batch_packed_tiles(cuda, T):
    """The matrix-core decode batch on a pinned layer reads its experts from a
    copy in 16-row tiles made by the first call with packing on: the same
    bytes reordered, so the outputs equal the GGUF-row kernels' bit for bit,
    on the call that makes the copy and on the next one. The test layer
    leaves two experts unregistered (NULL in both tables)."""
    lib = _lib.load()
    shape = W.MoEShape("mdec-8e", 2048, 8, 4, 768, True, W.Q4_K, W.Q4_K, W.Q6_K)
    m = M.DeviceMoE(shape, 1, seed=61, unregistered={(0, 2), (0, 5)})
    x, hb = W.host_hidden(shape.d, T, 61)
    hbt = torch.from_numpy(hb).to(cuda)
    outs = []
    try:
        for packed in (0, 1, 1):
            _lib.check(lib.vireo_hip_set_packed(packed), "vireo_hip_set_packed")
            xt = torch.from_numpy(x).to(cuda)
            m.forward(0, xt, hbt)
            outs.append(xt.cpu().numpy())
    finally:
        lib.vireo_hip_set_packed(1)
    assert np.abs(outs[0] - x).max() > 0  # the layer contributed
    np.testing.assert_array_equal(outs[1].view(np.uint32), outs[0].view(np.uint32))
    np.testing.assert_array_equal(outs[2].view(np.uint32), outs[0].view(np.uint32))
    m.close()


def test_prefill_q8_fragments(cuda):
    """The matrix-core GEMMs of a call of 64+ tokens on a pinned Q8_0 layer
    read a copy of its experts in matrix-operand fragments (each lane's bytes
    of a 32-row, 64-column step together) made by the first call with
    packing on: the outputs equal the GGUF-row kernels' bit for bit, on that
    call and the next. Two experts are unregistered."""
    lib = _lib.load()
    shape = W.SHAPES["olmoe-q8_0"]
    m = M.DeviceMoE(shape, 1, seed=67, unregistered={(0, 3), (0, 40)})
    x, hb = W.host_hidden(shape.d, 130, 67)
    hbt = torch.from_numpy(hb).to(cuda)
    outs = []
    try:
        for packed in (0, 1, 1):
            _lib.check(lib.vireo_hip_set_packed(packed), "vireo_hip_set_packed")
            xt = torch.from_numpy(x).to(cuda)
            m.forward(0, xt, hbt)
            outs.append(xt.cpu().numpy())
    finally:
        lib.vireo_hip_set_packed(1)
    assert np.abs(outs[0] - x).max() > 0
    np.testing.assert_array_equal(outs[1].view(np.uint32), outs[0].view(np.uint32))
    np.testing.assert_array_equal(outs[2].view(np.uint32), outs[0].view(np.uint32))
    m.close()


@pytest.mark.parametrize("case", ["tiny_q4km", "tiny_q8", "olmoe_q8_0", "qwen3_q4_k_m"])
def test_golden_moe_on_gpu(cuda, case):
    g = golden(f"moe_{case}.npz")
    d, E, k, fe, renorm, gt, ut, dt = (int(v) for v in g["shape"])
    shape = W.MoEShape(case, d, E, k, fe, bool(renorm), gt, ut, dt)
    m = M.DeviceMoE(shape, 1, seed=int(g["seed"][0]))
    xt = torch.from_numpy(g["x"]).to(cuda)
    idx, _ = m.forward(0, xt, torch.from_numpy(g["hb"]).to(cuda), return_routing=True)
    check(f"golden {case}", g["x"], xt.cpu().numpy(), g["x_out"], idx.cpu().numpy(), g["idx"])
    m.close()


@pytest.mark.parametrize("name,plan,T", [("olmoe-q4_k_m", 0, 1), ("olmoe-q4_k_m", 2, 3), ("olmoe-q4_k_m", 0, 12),
                                         ("olmoe-q8_0", 0, 80)])
def test_unregistered_expert_is_skipped(cuda, oracle, path, name, plan, T):
    """An expert without slices contributes nothing: the one-token plan, the
    matrix-core decode batch, whose down kernel combines (its rows of y are
    zeros), and the bf16 GEMMs on packed Q8_0 fragments (the expert's tiles
    write nothing; the combine kernel skips its rows)."""
    path(plan)
    shape = W.SHAPES[name]
    x, hb = W.host_hidden(shape.d, T, 52)
    probe = M.DeviceMoE(shape, 1, seed=52)
    first = probe.route(0, torch.from_numpy(hb).to(cuda))[0].cpu().numpy()
    probe.close()
    drop = {(0, int(first[0, 0])), (0, int(first[0, 3]))}
    m = M.DeviceMoE(shape, 1, seed=52, unregistered=drop)
    m._unregistered = drop
    xt = torch.from_numpy(x[:T]).to(cuda)
    idx, _ = m.forward(0, xt, torch.from_numpy(hb[:T]).to(cuda), return_routing=True)
    xo, io, _, _ = oracle_layer(oracle, m, 0, x[:T], hb[:T])
    check(f"unregistered {name} plan={plan} T={T}", x[:T], xt.cpu().numpy(), xo, idx.cpu().numpy(), io,
          tol=TOL_BF16 if T >= 64 else TOL)
    m.close()


def test_zero_tokens_is_a_no_op(cuda):
    shape = W.SHAPES["olmoe-q8_0"]
    m = M.DeviceMoE(shape, 1, seed=53)
    xt = torch.zeros((0, shape.d), dtype=torch.float32, device=cuda)
    m.forward(0, xt, xt)
    m.close()


def test_deterministic_and_batch_invariant(cuda, path):
    """No float atomics: the same call gives the same bits; on the grouped
    plan a token's result does not depend on the other tokens of its call as
    long as the calls run on the same kernels - 3 to 63 tokens on the matrix
    cores (16 tokens against two calls of 8, and 3 tokens against the same
    tokens in the 16), fewer than 3 on the fp32 decode-batch kernels (2
    tokens against single tokens). Across the switch the last bits differ,
    both within the parity tolerance."""
    shape = W.SHAPES["qwen3-30b-a3b-q4_k_m"]
    m = M.DeviceMoE(shape, 1, seed=54)
    x, hb = W.host_hidden(shape.d, 16, 54)
    hbt = torch.from_numpy(hb).to(cuda)

    def run(a, b):
        xt = torch.from_numpy(x[a:b].copy()).to(cuda)
        m.forward(0, xt, hbt[a:b].contiguous())
        return xt.cpu().numpy()

    outs = [run(0, 16) for _ in range(2)]
    np.testing.assert_array_equal(outs[0], outs[1])
    path(2)
    np.testing.assert_array_equal(np.concatenate([run(0, 8), run(8, 16)]), outs[0])
    np.testing.assert_array_equal(run(5, 8), outs[0][5:8])
    two = run(4, 6)
    for t in (4, 5):
        np.testing.assert_array_equal(run(t, t + 1)[0], two[t - 4])
    m.close()


def test_layers_are_independent(cuda, oracle):
    """A multi-layer model: each layer routes with its own router and experts."""
    shape = W.SHAPES["olmoe-q4_k_m"]
    m = M.DeviceMoE(shape, 3, seed=55)
    x, hb = W.host_hidden(shape.d, 1, 55)
    for layer in (2, 0):
        xt = torch.from_numpy(x).to(cuda)
        idx, _ = m.forward(layer, xt, torch.from_numpy(hb).to(cuda), return_routing=True)
        xo, io, _, _ = oracle_layer(oracle, m, layer, x, hb)
        check(f"layer {layer}", x, xt.cpu().numpy(), xo, idx.cpu().numpy(), io)
    m.close()


@pytest.mark.slow
def test_prefill_2048_zipf(cuda, oracle):
    """Qwen3-30B-A3B Q8_0 prefill of 2048 tokens under a Zipf(1.1) router
    bias: every token's experts bit-exact with the oracle and every token's
    output within the bf16 matrix-core tolerance (the oracle takes a few ms
    per token here, a few seconds for the call)."""
    shape = W.SHAPES["qwen3-30b-a3b-q8_0"]
    bias = W.zipf_bias(shape.E, 1.1, seed=7)
    m = M.DeviceMoE(shape, 1, seed=56, logit_bias=bias)
    T = 2048
    x, hb = W.host_hidden(shape.d, T, 56)
    xt = torch.from_numpy(x).to(cuda)
    idx, w = m.forward(0, xt, torch.from_numpy(hb).to(cuda), return_routing=True)
    ig = idx.cpu().numpy()
    router = m.host_router(0)
    oi = np.empty_like(ig)
    for t in range(T):
        lg = (oracle.matmul(W.F32, router, hb[t], shape.d, shape.E) + bias).astype(np.float32)
        oi[t] = oracle.topk(oracle.softmax(lg), shape.k, shape.renorm)[0]
    np.testing.assert_array_equal(ig, oi)
    xo, io, _, _ = oracle_layer(oracle, m, 0, x, hb)
    check("prefill, all 2048 tokens", x, xt.cpu().numpy(), xo, ig, io, tol=TOL_BF16)
    m.close()


def oracle_routing(oracle, m, hb, bias=None):
    shape = m.shape
    router = m.host_router(0)
    out = np.empty((len(hb), shape.k), dtype=np.int32)
    for t in range(len(hb)):
        lg = oracle.matmul(W.F32, router, hb[t], shape.d, shape.E)
        if bias is not None:
            lg = (lg + bias).astype(np.float32)
        out[t] = oracle.topk(oracle.softmax(lg), shape.k, shape.renorm)[0]
    return out


# (model, tokens, Zipf router bias): groups of >= 16 tokens (several 128-row
# tiles, ragged last tiles under the bias) next to smaller groups
MFMA_CASES = [("qwen3-30b-a3b-q8_0", 512, True), ("olmoe-q4_k_m", 128, False), ("qwen3-30b-a3b-q4_k_m", 128, False)]


@pytest.mark.parametrize("name,T,zipf", MFMA_CASES)
@pytest.mark.parametrize("plan", [0, 4])
def test_grouped_plan_large_groups(cuda, oracle, path, name, T, zipf, plan):
    """Calls of >= 64 tokens with groups of every size (1-15 tokens, and 16 to
    over 128): under plan 0 every group runs as bf16 matrix-core GEMMs, one
    tile or several, ragged or not; plan 4 runs all of them on the fp32
    kernels. Every token's experts bit-exact and every token's output
    against the oracle; the same call twice gives the same bits."""
    path(plan)
    shape = W.SHAPES[name]
    bias = W.zipf_bias(shape.E, 1.1, seed=8) if zipf else None
    m = M.DeviceMoE(shape, 1, seed=59, logit_bias=bias)
    x, hb = W.host_hidden(shape.d, T, 59)
    hbt = torch.from_numpy(hb).to(cuda)
    outs = []
    for _ in range(2):
        xt = torch.from_numpy(x).to(cuda)
        idx, _ = m.forward(0, xt, hbt, return_routing=True)
        outs.append(xt.cpu().numpy())
    np.testing.assert_array_equal(outs[0], outs[1])
    ig = idx.cpu().numpy()
    np.testing.assert_array_equal(ig, oracle_routing(oracle, m, hb, bias))
    counts = np.bincount(ig.ravel(), minlength=shape.E)
    assert counts.max() >= 16 and ((counts > 0) & (counts < 16)).any(), counts
    if zipf:
        assert counts.max() > 128, counts.max()
    xo, io, _, _ = oracle_layer(oracle, m, 0, x, hb)
    check(f"{name} T={T} plan={plan}", x, outs[0], xo, ig, io, tol=TOL_BF16 if plan == 0 else TOL)
    m.close()


def test_grouped_plan_large_groups_unregistered(cuda, oracle, path):
    """Unregistered experts among the matrix-core groups contribute nothing."""
    path(0)
    shape = W.SHAPES["olmoe-q4_k_m"]
    T = 256
    x, hb = W.host_hidden(shape.d, T, 60)
    probe = M.DeviceMoE(shape, 1, seed=60)
    ig = probe.route(0, torch.from_numpy(hb).to(cuda))[0].cpu().numpy()
    probe.close()
    counts = np.bincount(ig.ravel(), minlength=shape.E)
    big = np.argsort(-counts, kind="stable")
    drop = {(0, int(big[0])), (0, int(big[5]))}
    m = M.DeviceMoE(shape, 1, seed=60, unregistered=drop)
    m._unregistered = drop
    xt = torch.from_numpy(x).to(cuda)
    idx, _ = m.forward(0, xt, torch.from_numpy(hb).to(cuda), return_routing=True)
    assert (ig == big[0]).any(axis=1).sum() >= 16  # the dropped expert had a matrix-core group
    xo, io, _, _ = oracle_layer(oracle, m, 0, x, hb)
    check("unregistered large groups, all tokens", x, xt.cpu().numpy(), xo, idx.cpu().numpy(), io, tol=TOL_BF16)
    m.close()


@pytest.mark.parametrize("plan", [0, 3])
@pytest.mark.parametrize("name", ["qwen3-30b-a3b-q4_k_m", "olmoe-q8_0", "olmoe-q4_k_m"])
def test_decode_stages_equal_forward(cuda, path, name, plan):
    """moe_decode_stage 0, 1, 2 over a caller-owned state gives
    moe_ffn_forward's single-token result bit for bit (three-kernel and fused)."""
    path(plan)
    shape = W.SHAPES[name]
    m = M.DeviceMoE(shape, 2, seed=57)
    x, hb = W.host_hidden(shape.d, 1, 57)
    hbt = torch.from_numpy(hb).to(cuda)
    for layer in (1, 0):
        xa = torch.from_numpy(x).to(cuda)
        ia, wa = m.forward(layer, xa, hbt, return_routing=True)
        xb = torch.from_numpy(x).to(cuda)
        state = m.decode_state()
        ib = torch.empty_like(ia)
        wb = torch.empty_like(wa)
        for stage in range(3):
            m.decode_stage(layer, stage, xb[0], hbt[0], state, ib, wb)
        np.testing.assert_array_equal(xb.cpu().numpy(), xa.cpu().numpy())
        np.testing.assert_array_equal(ib.cpu().numpy(), ia.cpu().numpy())
        np.testing.assert_array_equal(wb.cpu().numpy(), wa.cpu().numpy())
    m.close()


@pytest.mark.parametrize("plan", [1, 3, 5])
@pytest.mark.parametrize("name", ["olmoe-q8_0", "qwen3-30b-a3b-q4_k_m"])
def test_decode_plan_ties_take_the_exact_path(cuda, oracle, path, name, plan):
    """Exactly tied router rows inside and at the edge of the top-k: the
    decode kernel's one-wave ranking cannot certify the order and the whole
    workgroup re-ranks on exact logits; experts and output match the oracle."""
    path(plan)
    shape = W.SHAPES[name]
    m = M.DeviceMoE(shape, 1, seed=58)
    r = m.routers[0]
    x, hb = W.host_hidden(shape.d, 1, 58)
    order = np.argsort(-(m.host_router(0) @ hb[0]), kind="stable")
    for a, b in ((order[0], order[1]), (order[7], order[8]), (order[3], order[20])):
        r[b].copy_(r[a])  # b now ties a exactly
    xt = torch.from_numpy(x).to(cuda)
    idx, w = m.forward(0, xt, torch.from_numpy(hb).to(cuda), return_routing=True)
    xo, io, wo, _ = oracle_layer(oracle, m, 0, x, hb)
    check(f"{name} decode ties", x, xt.cpu().numpy(), xo, idx.cpu().numpy(), io)
    np.testing.assert_allclose(w.cpu().numpy(), wo, rtol=1e-5)
    state = m.decode_state()
    ib, wb = torch.empty_like(idx), torch.empty_like(w)
    xs = torch.from_numpy(x).to(cuda)
    hbt = torch.from_numpy(hb).to(cuda)
    for stage in range(3):
        m.decode_stage(0, stage, xs[0], hbt[0], state, ib, wb)
    flags = state[-256:].view(torch.int32)  # the flag word is the state's last 256-byte slot
    assert int(flags[0].cpu()) & 2, "near tie not reported"
    m.close()


@pytest.mark.parametrize("name", ["qwen3-30b-a3b-q4_k_m", "olmoe-q8_0", "olmoe-q4_k_m", "qwen3-30b-a3b-q8_0"])
def test_layer_kernel_sequence(cuda, oracle, path, name):
    """Plan 5 runs the whole one-token layer in one launch whose workgroups
    meet through records tagged with the launch's number: many calls in a
    row, over two layers and distinct tokens, each matching the oracle and
    the separate-kernel plan (the same decoders and combine order; the router
    sums may differ in their last fp64 bits)."""
    shape = W.SHAPES[name]
    m = M.DeviceMoE(shape, 2, seed=62)
    n = 12
    x, hb = W.host_hidden(shape.d, n, 62)
    hbt = torch.from_numpy(hb).to(cuda)
    outs = {}
    for plan in (1, 5):
        path(plan)
        xs = torch.from_numpy(x).to(cuda)
        ids = []
        for t in range(n):
            idx, _ = m.forward(t % 2, xs[t:t + 1], hbt[t:t + 1], return_routing=True)
            ids.append(idx.cpu().numpy()[0])
        outs[plan] = (xs.cpu().numpy(), np.array(ids))
    for layer in (0, 1):
        sel = np.arange(layer, n, 2)
        xo, io, _, _ = oracle_layer(oracle, m, layer, x, hb, tokens=sel)
        check(f"{name} plan 5 layer {layer}", x[sel], outs[5][0][sel], xo, outs[5][1][sel], io)
    np.testing.assert_array_equal(outs[5][1], outs[1][1])
    d5, d1 = outs[5][0] - x, outs[1][0] - x
    assert np.abs(d5 - d1).max() <= 1e-5 * np.abs(d1).max()
    m.close()


@pytest.mark.parametrize("name", ["qwen3-30b-a3b-q4_k_m", "olmoe-q8_0"])
def test_decode_phases_stamps(cuda, name):
    """moe_decode_phases: the same results as moe_ffn_forward bit for bit, and
    for every call three kernels whose workgroups' stamps never go backwards,
    each kernel starting after the previous one's phases (stream order)."""
    shape = W.SHAPES[name]
    m = M.DeviceMoE(shape, 2, seed=64)
    n = 6
    x, hb = W.host_hidden(shape.d, n, 64)
    hbt = torch.from_numpy(hb).to(cuda)
    xs = torch.from_numpy(x).to(cuda)
    layers = [t % 2 for t in range(n)]
    st = m.decode_phases(layers, xs, hbt)
    torch.cuda.synchronize()
    xr = torch.from_numpy(x).to(cuda)
    for t in range(n):
        m.forward(layers[t], xr[t:t + 1], hbt[t:t + 1])
    torch.cuda.synchronize()
    assert torch.equal(xs, xr)
    stamps = st.cpu().numpy().reshape(n, 3, 256, 8)
    nphase = {0: 2, 1: 5, 2: 5}
    for call in stamps:
        prev_end = 0
        for kk in range(3):
            wg = call[kk][call[kk][:, 0] > 0]
            assert len(wg) > 0, f"kernel {kk} recorded nothing"
            ph = wg[:, :nphase[kk]]
            assert (np.diff(ph, axis=1) >= 0).all(), f"kernel {kk}: a stamp went backwards"
            assert wg[:, 0].min() >= prev_end
            prev_end = ph.max()
    m.close()
