"""The 48-layer Qwen3-30B-A3B-shaped MoE stack at full size on the GPU
(128 experts per layer, top-8 renormalised, d=2048, fe=768, gate/up Q4_K,
down Q6_K; a [151936 x 2048] Q8_0 LM head, tied; about 19 GB in HBM) against
the oracle's restatement of the reference's decode skeleton
(src/gguf_run.c:216-254 with attention omitted), step after step.

The steps are chained greedily: each step's input token is the GPU's
argmax of the step before, from one random first token.
moe_stack_step_trace records every layer's routing. For each step the oracle
runs its own trajectory from the same input token: x = embedding row, then per layer xb = rmsnorm(x),
the router logits, softmax and top-8 (its own routing), moe_ffn on those
experts; then the final norm, the LM head and argmax. Only the router and the
8 routed experts' slices of each layer are copied from HBM for the oracle
(the whole model is never rebuilt on the host).

Bar: every layer's expert ids equal the oracle's in selection order, except
at a near tie: the oracle's exact logit gap at a selection boundary below
1e-6, or a layer the GPU flagged (its fp64 bound could not separate two
logits, so their order rests on the fp32 rounding of the reference's sum,
or its exact gap was below 1e-6). The two trajectories differ by fp32
rounding (about 3e-5 of x after 30 layers), which is enough to flip such an
order; where the two orders differ, the experts' oracle logits must be
within 1e-4 of the largest logit. A near tie is counted and ends the
comparison of that step's later
layers (the trajectories part there), at most MAX_NEAR such steps per run; residual and logits within 2e-3 of their largest
magnitude; tokens equal unless the oracle's top two logits are closer than
that.
"""
import numpy as np
import pytest
import torch

from vireo_amd import stack as S
from vireo_amd import workloads as W

pytestmark = [pytest.mark.gpu, pytest.mark.slow]
TOL = 2e-3
NEAR_TIE = 1e-6
ROUTE_EXACT = 1
ROUTE_NEAR_TIE = 2
MAX_NEAR = 8  # of 32 steps
FLIP = 1e-4  # a flipped order's logit difference, relative to the largest logit


def oracle_routing(oracle, shape, router, xb):
    """The reference's routing of one token (src/gguf_run.c:187-192): ids in
    selection order, the smallest exact logit gap that decides them, and the
    logits."""
    logits = oracle.matmul(W.F32, router, xb, shape.d, shape.E)
    idx, _ = oracle.topk(oracle.softmax(logits), shape.k, shape.renorm)
    order = np.sort(logits)[::-1]
    gaps = order[:shape.k] - order[1:shape.k + 1]
    return idx, float(gaps.min()), logits


@pytest.mark.parametrize("plan", [0, 5])
def test_stack48_full_size_matches_oracle(cuda, oracle, plan):
    from vireo_amd import _lib
    lib = _lib.load()
    shape = W.SHAPES["qwen3-30b-a3b-q4_k_m"]
    L, vocab, steps = 48, 151936, 32
    _lib.check(lib.vireo_hip_set_path(plan), "vireo_hip_set_path")
    st = None
    try:
        st = S.DeviceStack(shape, L, vocab=vocab, seed=2024)
        d, k = shape.d, shape.k
        lm = st.device_lm_head()
        rb = W.row_bytes(W.Q8_0, d)
        routers = [st.moe.host_router(l) for l in range(L)]
        ones = np.ones(d, np.float32)
        idx = torch.empty((L, k), dtype=torch.int32, device=cuda)
        flags = torch.empty(L, dtype=torch.int32, device=cuda)
        token = torch.empty(1, dtype=torch.int32, device=cuda)
        tok = int(np.random.default_rng(5).integers(0, vocab))
        compared = near = fallback = 0
        for step in range(steps):
            token.fill_(tok)
            st.step_trace(token, idx, flags)
            torch.cuda.synchronize()
            gi, gf = idx.cpu().numpy(), flags.cpu().numpy().astype(np.uint32)
            tg = int(token.cpu()[0])
            fallback += int(np.count_nonzero(gf & 1))
            x = oracle.dequant_row(W.Q8_0, lm[tok * rb:(tok + 1) * rb], d)
            parted = False
            for l in range(L):
                xb = oracle.rmsnorm(x, ones, W.EPS)
                oi, gap, lo = oracle_routing(oracle, shape, routers[l], xb)
                if not np.array_equal(gi[l], oi):
                    # where the two orders differ, the experts' oracle logits are within FLIP
                    diff = np.abs(lo[gi[l]] - lo[oi]).max() / np.abs(lo).max()
                    assert (gap < NEAR_TIE or (gf[l] & (ROUTE_EXACT | ROUTE_NEAR_TIE))) and diff <= FLIP, \
                        f"step {step} layer {l}: GPU experts {gi[l]} vs oracle {oi} (gap {gap:.3e}, flags {gf[l]}, " \
                        f"logit difference {diff:.3e})"
                    near += 1
                    parted = True
                    break
                compared += 1
                experts = {int(e): st.moe.expert_bytes(l, int(e)) for e in oi}
                G = [experts[e][0] if e in experts else None for e in range(shape.E)]
                U = [experts[e][1] if e in experts else None for e in range(shape.E)]
                D = [experts[e][2] if e in experts else None for e in range(shape.E)]
                x, io, _, _ = oracle.moe_ffn(shape, routers[l], G, U, D, x, xb)
                x = x[0]
                assert np.array_equal(io[0], oi)
            if not parted:
                logits = oracle.matmul(W.Q8_0, lm, oracle.rmsnorm(x, ones, W.EPS), d, vocab)
                xg, lg = st.x.cpu().numpy(), st.logits.cpu().numpy()
                rx = np.abs(xg - x).max() / np.abs(x).max()
                rl = np.abs(lg - logits).max() / np.abs(logits).max()
                to = oracle.argmax(logits)
                print(f"step {step}: token {tok} -> {tg} (oracle {to}); x {rx:.2e}, logits {rl:.2e}", flush=True)
                assert rx <= TOL and rl <= TOL
                top2 = np.sort(logits)[-2:]
                if top2[1] - top2[0] > TOL * np.abs(logits).max():
                    assert tg == to
            tok = tg  # greedy: the next step reads this step's token
        print(f"{compared} layer routings equal to the oracle's, {near} near ties, {fallback} exact-logit fallbacks")
        assert near <= MAX_NEAR
        assert compared >= L * (steps - near)
    finally:
        if st is not None:
            st.close()
        lib.vireo_hip_set_path(0)
