"""moe_stack_step on the GPU against the oracle's restatement of the
reference's decode skeleton (src/gguf_run.c:216-254 with attention omitted):
x = embedding row of the token (the tied Q8_0 LM head, :218 / :297); per
layer xb = rmsnorm(x) (:161-165, unit weight) and moe_ffn adds to x
(:185-214); logits = LM head * rmsnorm(x) (:249-250); token = argmax (:254).

Bar: the residual and the logits within 2e-3 of their largest magnitude after
every step, the greedy tokens equal (unless the top two logits of the oracle
are closer than the tolerance). With a tied random LM head a token's own row
dominates its logits, so greedy decoding would repeat one token; the steps
are fed a sequence of distinct tokens instead, through the device token
buffer the step reads.
"""
import numpy as np
import pytest
import torch

from conftest import expert_lists
from vireo_amd import stack as S
from vireo_amd import workloads as W

pytestmark = pytest.mark.gpu
TOL = 2e-3


def oracle_stack(oracle, st):
    shape, d = st.shape, st.shape.d
    lm = st.host_lm_head()
    rb = W.row_bytes(st.lm_type, d)
    layers = [expert_lists(shape, *st.moe.host_layer(l)) for l in range(st.n_layers)]
    routers = [st.moe.host_router(l) for l in range(st.n_layers)]
    ones = np.ones(d, np.float32)

    def step(tok):
        x = oracle.dequant_row(st.lm_type, lm[tok * rb:(tok + 1) * rb], d)
        for l in range(st.n_layers):
            xb = oracle.rmsnorm(x, ones, W.EPS)
            x = oracle.moe_ffn(shape, routers[l], *layers[l], x, xb)[0][0]
        logits = oracle.matmul(st.lm_type, lm, oracle.rmsnorm(x, ones, W.EPS), d, st.vocab)
        return x, logits, oracle.argmax(logits)
    return step


@pytest.mark.parametrize("name,plan", [("qwen3-16e", 0), ("qwen3-16e", 5), ("tiny", 0)])
def test_stack_decode_matches_oracle(cuda, oracle, name, plan):
    """qwen3-16e: Qwen3-30B-A3B layers (Q4_K / Q6_K, d=2048, fe=768, top-8
    renormalised) with 16 experts each, on the one-token decode plan (plan 0)
    and on the whole-layer kernel with the RMSNorm fused in (plan 5); tiny:
    d=256 layers, which take the grouped plan."""
    if name == "qwen3-16e":
        shape = W.SHAPES["qwen3-30b-a3b-q4_k_m"].with_(name=name, E=16)
        n_layers, vocab = 3, 4096
    else:
        shape = W.MoEShape(name, 256, 8, 2, 256, True, W.Q4_K, W.Q4_K, W.Q6_K)
        n_layers, vocab = 4, 1000
    from vireo_amd import _lib
    lib = _lib.load()
    _lib.check(lib.vireo_hip_set_path(plan), "vireo_hip_set_path")
    st = S.DeviceStack(shape, n_layers, vocab=vocab, seed=61)
    ref = oracle_stack(oracle, st)
    token = torch.empty(1, dtype=torch.int32, device=cuda)
    for i, tok in enumerate((17, vocab - 1, vocab // 3, 0)):
        token.fill_(tok)
        st.step(token)
        xo, lo, to = ref(tok)
        xg, lg, tg = st.x.cpu().numpy(), st.logits.cpu().numpy(), int(token.cpu()[0])
        rx = np.abs(xg - xo).max() / np.abs(xo).max()
        rl = np.abs(lg - lo).max() / np.abs(lo).max()
        print(f"{name} step {i}: token {tok} -> {tg} (oracle {to}); x max rel {rx:.2e}, logits max rel {rl:.2e}")
        assert rx <= TOL and rl <= TOL
        top2 = np.sort(lo)[-2:]
        if top2[1] - top2[0] > TOL * np.abs(lo).max():
            assert tg == to
    st.close()
    lib.vireo_hip_set_path(0)


def test_embed_rows_and_range(cuda, oracle):
    """vireo_embed: rows of a Q8_0 table by device token ids equal the
    reference's gguf_dequant_row of those rows bit for bit; an id outside the
    table gives a zero row."""
    import ctypes as C
    from vireo_amd import _lib
    lib = _lib.load()
    d, rows = 256, 50
    tab = W.host_matrix(W.Q8_0, d, 0, rows, 62, W.stream_id(0, W.KIND_LM_HEAD))
    tab_d = torch.from_numpy(tab).to(cuda)
    ids = torch.tensor([0, 49, 7, -1, 50, 7], dtype=torch.int32, device=cuda)
    out = torch.empty((6, d), dtype=torch.float32, device=cuda)
    _lib.check(lib.vireo_embed(W.Q8_0, C.c_void_p(tab_d.data_ptr()), d, rows, C.c_void_p(ids.data_ptr()), 6,
                               C.c_void_p(out.data_ptr()), None), "vireo_embed")
    got = out.cpu().numpy()
    rb = W.row_bytes(W.Q8_0, d)
    for i, t in enumerate([0, 49, 7, -1, 50, 7]):
        want = oracle.dequant_row(W.Q8_0, tab[t * rb:(t + 1) * rb], d) if 0 <= t < rows else np.zeros(d, np.float32)
        np.testing.assert_array_equal(got[i], want)
