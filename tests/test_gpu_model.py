"""Whole-model decode (vireo_model_step) against the reference's own forward()
(src/gguf_run.c:216-251, compiled from its sources into oracle/_ref) on the
same synthetic GGUF files.

Each case writes a small model (two or three blocks, d=256, grouped-query
attention with head size 64) and feeds the same token sequence to both: a
prompt of 5 tokens (logits only at its last position, as the reference runner
does) and then greedy decoding up to 20 positions, so the KV store crosses
several blocks of 4 tokens. At every position the residual stream after the
last block, and the logits where computed, agree within 2e-3 of their largest
magnitude; the greedy token agrees unless the reference's two best logits are
within 1e-4 of the largest logit (then both continue with the reference's
token, and the case is counted). Cases cover:

* MoE blocks (Qwen3: per-head QK-norm, renormalised top-k; OLMoE: QK-norm
  over the whole vector, raw top-k probabilities, Q8_0 experts);
* dense SwiGLU blocks with q/k/v biases, no QK-norm, the default head size
  dim / heads, F16 norm weights (dequantized at load), Q5_0 attention and
  F16 / Q8_0 / Q6_K FFN matrices, an untied head;
* a tied head (the LM head is the token embedding) with F32 attention and
  Q4_K FFN matrices;
* Q4_K and Q6_K attention matrices.
"""
import numpy as np
import pytest
import torch

from vireo_amd import gguf as G
from vireo_amd import workloads as W

pytestmark = pytest.mark.gpu
TOL = 2e-3
BLOCK = 4
PROMPT = [3, 17, 250, 9, 101]
STEPS = 20

CASES = {
    "qwen3moe": dict(arch="qwen3moe", n_layers=2, d=256, n_heads=8, n_kv_heads=2, head_size=64, vocab=512,
                     moe=W.MoEShape("m", 256, 8, 2, 256, True, W.Q4_K, W.Q4_K, W.Q6_K), qk_norm="head",
                     untied=True),
    "olmoe": dict(arch="olmoe", n_layers=2, d=256, n_heads=4, n_kv_heads=4, head_size=64, vocab=384,
                  moe=W.MoEShape("o", 256, 8, 3, 256, False, W.Q8_0, W.Q8_0, W.Q8_0), qk_norm="full",
                  untied=True, explicit_head=False),
    "qwen2-dense": dict(arch="qwen2", n_layers=3, d=256, n_heads=4, n_kv_heads=2, head_size=64, vocab=512, ffn=512,
                        bias=True, qk_norm=None, explicit_head=False, attn_type=W.Q5_0,
                        ffn_types=(W.F16, W.Q8_0, W.Q6_K), norm_type=W.F16, untied=True),
    "llama-tied": dict(arch="llama", n_layers=2, d=256, n_heads=4, n_kv_heads=1, head_size=64, vocab=256, ffn=256,
                       qk_norm=None, explicit_head=False, attn_type=W.F32, ffn_types=(W.Q4_K, W.Q4_K, W.Q4_K)),
    # K-quant attention matrices (q, k and v on the register-resident decoders)
    "llama-q4k-attn": dict(arch="llama", n_layers=2, d=256, n_heads=4, n_kv_heads=2, head_size=64, vocab=256,
                           ffn=256, qk_norm=None, explicit_head=False, attn_type=W.Q4_K,
                           ffn_types=(W.Q8_0, W.Q8_0, W.Q8_0)),
    "olmoe-q6k-attn": dict(arch="olmoe", n_layers=2, d=256, n_heads=4, n_kv_heads=4, head_size=64, vocab=384,
                           moe=W.MoEShape("o", 256, 8, 3, 256, False, W.Q4_K, W.Q4_K, W.Q6_K), qk_norm="full",
                           untied=True, explicit_head=False, attn_type=W.Q6_K),
}


@pytest.fixture(scope="module")
def ref():
    from oracle.oracle import Reference
    if not Reference.available():
        pytest.skip("oracle/_ref not built")
    return Reference()


def rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("name", list(CASES))
def test_decode_matches_reference_forward(cuda, ref, tmp_path, name):
    from oracle.oracle import RefModel
    from vireo_amd.model import GGUFDecoder
    cfg = dict(CASES[name])
    path = tmp_path / f"{name}.gguf"
    G.write_model_gguf(str(path), seed=41, **cfg)
    r = RefModel(ref, path, block_tokens=BLOCK)
    g = GGUFDecoder(path, max_pos=64, block_tokens=BLOCK)
    assert (g.dim, g.vocab, g.n_layers, g.n_heads, g.n_kv_heads, g.head_size, g.is_moe) == (
        r.dim, r.vocab, r.n_layers, r.n_heads, r.n_kv_heads, r.head_size, bool(r.is_moe))
    tok, near, worst_x, worst_l, seq = PROMPT[0], 0, 0.0, 0.0, []
    for pos in range(STEPS):
        want = pos >= len(PROMPT) - 1
        xr, lr = r.forward(tok, pos, want)
        nt = g.step(tok, pos, want)
        torch.cuda.synchronize()
        worst_x = max(worst_x, rel(g.x.cpu().numpy(), xr))
        if want:
            worst_l = max(worst_l, rel(g.logits.cpu().numpy(), lr))
            top2 = np.sort(lr)[-2:]
            ref_tok = int(np.argmax(lr))
            if nt != ref_tok:
                assert top2[1] - top2[0] < 1e-4 * np.abs(lr).max(), (pos, nt, ref_tok)
                near += 1
            tok = ref_tok
            seq.append(tok)
        else:
            tok = PROMPT[pos + 1]
    print(f"{name}: residual max rel {worst_x:.2e}, logits max rel {worst_l:.2e}, near ties {near}, "
          f"tokens {seq}")
    if cfg.get("untied"):  # with the embedding as its head, a tied model repeats its input token here
        assert len(set(seq)) > 1
    assert worst_x <= TOL and worst_l <= TOL
    g.close()
    r.close()


def test_rope_table_is_the_reference_expression(cuda, lib):
    """Row p, column j < hs/2: cosf(p * powf(base, -2j/hs)); then the sines
    (src/gguf_run.c:171-172), evaluated on the host by the C library."""
    import ctypes as C
    hs, P, base = 64, 40, 1.0e6
    t = torch.empty((P, hs), dtype=torch.float32, device=cuda)
    assert lib.vireo_rope_table(C.c_float(base), hs, P, C.c_void_p(t.data_ptr())) == 0
    tab = t.cpu().numpy().astype(np.float64)
    # exact angles p * base^(-2j/hs); the float expression rounds the exponent,
    # powf and the product (each within an ulp), so |da| <= 4 * 2^-24 * a, and
    # cosf / sinf add half an ulp
    a = np.arange(P, dtype=np.float64)[:, None] * np.power(base, -2.0 * np.arange(hs // 2) / hs)[None, :]
    bound = 4 * 2.0 ** -24 * a + 2.0 ** -24
    assert (np.abs(tab[:, :hs // 2] - np.cos(a)) <= bound).all()
    assert (np.abs(tab[:, hs // 2:] - np.sin(a)) <= bound).all()
    assert lib.vireo_rope_table(C.c_float(base), 63, P, C.c_void_p(t.data_ptr())) < 0


def test_model_step_rejects_positions_past_the_table(cuda, tmp_path):
    from vireo_amd import _lib
    from vireo_amd.model import GGUFDecoder
    path = tmp_path / "m.gguf"
    G.write_model_gguf(str(path), seed=5, **CASES["llama-tied"])
    g = GGUFDecoder(path, max_pos=8, block_tokens=BLOCK)
    g.step(1, 0, False)
    with pytest.raises(_lib.VireoError):
        g.step(1, 8, True)
    g.close()


def test_model_load_names_what_is_missing(cuda, tmp_path):
    from vireo_amd import _lib
    from vireo_amd.model import GGUFDecoder
    w = G.GGUFWriter()
    w.add("general.architecture", G.STRING, "llama")
    w.add("llama.block_count", G.U32, 1)
    w.add("llama.embedding_length", G.U32, 256)
    w.add("llama.feed_forward_length", G.U32, 256)
    w.add("llama.attention.head_count", G.U32, 4)
    w.add("llama.attention.head_count_kv", G.U32, 4)
    w.add_tensor("blk.0.attn_norm.weight", [256], W.F32, np.ones(256, np.float32))
    path = tmp_path / "broken.gguf"
    w.write(str(path))
    with pytest.raises(_lib.VireoError, match="attn_q"):
        GGUFDecoder(path, max_pos=8)


@pytest.mark.parametrize("name", ["qwen3moe", "qwen2-dense"])
def test_device_position_steps_and_graph(cuda, tmp_path, name):
    """vireo_model_step_pos (position on the device, contiguous KV store) gives
    vireo_model_step's results bit for bit; and a greedy continuation captured
    in one HIP graph (the device position advancing inside) replays to the same
    tokens and logits as the same steps run eagerly."""
    from vireo_amd.model import GGUFDecoder
    path = tmp_path / f"{name}.gguf"
    G.write_model_gguf(str(path), seed=43, **CASES[name])
    host = GGUFDecoder(path, max_pos=64, block_tokens=BLOCK)
    devp = GGUFDecoder(path, max_pos=64, block_tokens=BLOCK, contiguous=True)
    tok = PROMPT[0]
    for pos in range(12):  # prompt, then greedy
        want = pos >= len(PROMPT) - 1
        nt = host.step(tok, pos, want)
        devp.token.fill_(tok)
        devp.step_pos(want)
        torch.cuda.synchronize()
        assert torch.equal(host.x, devp.x), pos
        if want:
            assert torch.equal(host.logits, devp.logits), pos
            assert int(devp.token.item()) == nt
        tok = nt if want else PROMPT[pos + 1]
    assert int(devp.pos.item()) == 12
    # eager reference continuation on the host-position decoder
    start, eager = tok, []
    for pos in range(12, 20):
        tok = host.step(tok, pos, True)
        eager.append((tok, host.logits.clone()))
    # the same 8 steps captured once (nothing runs while capturing) and replayed
    assert int(devp.token.item()) == start
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    logits = []
    with torch.cuda.graph(g, stream=s):
        for _ in range(8):
            devp.step_pos(True, stream=s)
            logits.append(devp.logits.clone())
    torch.cuda.synchronize()
    assert int(devp.pos.item()) == 12
    g.replay()
    torch.cuda.synchronize()
    for i, (t, lg) in enumerate(eager):
        assert torch.equal(logits[i], lg), i
    assert int(devp.token.item()) == eager[-1][0] and int(devp.pos.item()) == 20
    host.close()
    devp.close()
