"""The MoE layer shapes the path is measured on, and their synthetic inputs.

Shapes (hidden d, experts E, top-k, expert intermediate fe, renorm, types):
  olmoe-q8_0          OLMoE-1B-7B: d=2048, E=64,  k=8, fe=1024, no renorm, Q8_0 / Q8_0 / Q8_0
  olmoe-q4_k_m        OLMoE-1B-7B: d=2048, E=64,  k=8, fe=1024, no renorm, Q4_K / Q4_K / Q6_K
  qwen3-30b-a3b-q4_k_m  Qwen3-30B-A3B: d=2048, E=128, k=8, fe=768, renorm, Q4_K / Q4_K / Q6_K
  qwen3-30b-a3b-q8_0  Qwen3-30B-A3B: d=2048, E=128, k=8, fe=768, renorm, Q8_0 / Q8_0 / Q8_0

Renormalisation follows the reference rule topk_renorm = (arch != "olmoe")
(src/gguf_run.c:292). Every value is deterministic in (seed, layer, tensor):
expert weights are N(0, 0.02) then quantized, routers F32 N(0, 0.02), hidden
states N(0, 1) then RMSNorm'd with unit weight and eps 1e-6. Stacked expert
tensors are laid out as GGUF stores ffn_{gate,up,down}_exps: expert e's slice
of a [E x rows x cols] tensor is rows [e*rows, (e+1)*rows).
"""
import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib

F32, F16, Q5_0, Q8_0, Q4_K, Q6_K = 0, 1, 6, 8, 12, 14
TYPE_NAMES = {F32: "F32", F16: "F16", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}
BLOCK = {F32: (1, 4), F16: (1, 2), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}

KIND_ROUTER, KIND_GATE, KIND_UP, KIND_DOWN, KIND_HIDDEN, KIND_LM_HEAD, KIND_BIAS = range(7)
EPS = 1e-6
WEIGHT_SIGMA = 0.02


@dataclass(frozen=True)
class MoEShape:
    name: str
    d: int
    E: int
    k: int
    fe: int
    renorm: bool
    gate_type: int
    up_type: int
    down_type: int

    def slice_bytes(self):
        """Bytes of one expert's gate, up and down slices."""
        return (row_bytes(self.gate_type, self.d) * self.fe, row_bytes(self.up_type, self.d) * self.fe,
                row_bytes(self.down_type, self.fe) * self.d)

    def expert_bytes(self):
        return sum(self.slice_bytes())

    def with_(self, **kw):
        f = dict(self.__dict__)
        f.update(kw)
        return MoEShape(**f)


SHAPES = {
    "olmoe-q8_0": MoEShape("olmoe-q8_0", 2048, 64, 8, 1024, False, Q8_0, Q8_0, Q8_0),
    "olmoe-q4_k_m": MoEShape("olmoe-q4_k_m", 2048, 64, 8, 1024, False, Q4_K, Q4_K, Q6_K),
    "qwen3-30b-a3b-q4_k_m": MoEShape("qwen3-30b-a3b-q4_k_m", 2048, 128, 8, 768, True, Q4_K, Q4_K, Q6_K),
    "qwen3-30b-a3b-q8_0": MoEShape("qwen3-30b-a3b-q8_0", 2048, 128, 8, 768, True, Q8_0, Q8_0, Q8_0),
}
LM_VOCAB = 151936


def row_bytes(typ, n):
    be, bb = BLOCK[typ]
    assert n % be == 0, (typ, n)
    return n // be * bb


def stream_id(layer, kind):
    return layer * 16 + kind


def _vp(a):
    return a.ctypes.data_as(C.c_void_p)


def host_matrix(typ, n, first_row, rows, seed, stream, sigma=WEIGHT_SIGMA):
    """Rows [first_row, first_row+rows) of a synthetic quantized matrix (bytes)."""
    out = np.empty(row_bytes(typ, n) * rows, np.uint8)
    _lib.check(_lib.load().vireo_synth_matrix(typ, _vp(out), n, first_row, rows, seed, stream, sigma),
               "vireo_synth_matrix")
    return out


def host_normal(count, seed, stream, first=0, sigma=1.0):
    out = np.empty(count, np.float32)
    _lib.check(_lib.load().vireo_synth_normal(_vp(out), count, seed, stream, first, sigma), "vireo_synth_normal")
    return out


def host_router(shape, layer, seed):
    return host_normal(shape.E * shape.d, seed, stream_id(layer, KIND_ROUTER), sigma=WEIGHT_SIGMA).reshape(
        shape.E, shape.d)


def host_expert(shape, layer, e, seed):
    """(gate, up, down) byte arrays of expert e of `layer`."""
    return (host_matrix(shape.gate_type, shape.d, e * shape.fe, shape.fe, seed, stream_id(layer, KIND_GATE)),
            host_matrix(shape.up_type, shape.d, e * shape.fe, shape.fe, seed, stream_id(layer, KIND_UP)),
            host_matrix(shape.down_type, shape.fe, e * shape.d, shape.d, seed, stream_id(layer, KIND_DOWN)))


def host_layer(shape, layer, seed):
    """Stacked (gate_all, up_all, down_all) for all E experts of `layer`."""
    E = shape.E
    return (host_matrix(shape.gate_type, shape.d, 0, E * shape.fe, seed, stream_id(layer, KIND_GATE)),
            host_matrix(shape.up_type, shape.d, 0, E * shape.fe, seed, stream_id(layer, KIND_UP)),
            host_matrix(shape.down_type, shape.fe, 0, E * shape.d, seed, stream_id(layer, KIND_DOWN)))


def host_hidden(d, tokens, seed, stream=stream_id(0, KIND_HIDDEN), eps=EPS):
    """(x, hb): N(0,1) hidden states and their unit-weight RMSNorm."""
    x = np.empty((tokens, d), np.float32)
    hb = np.empty((tokens, d), np.float32)
    _lib.check(_lib.load().vireo_synth_hidden(_vp(x), _vp(hb), d, tokens, seed, stream, eps), "vireo_synth_hidden")
    return x, hb


def zipf_bias(E, s=1.1, seed=0):
    """Per-expert router logit bias log(p) of a Zipf(s) law over E ranks; the
    rank of each expert is a seeded permutation."""
    ranks = np.arange(1, E + 1, dtype=np.float64)
    p = ranks ** (-s)
    p /= p.sum()
    perm = np.random.default_rng(seed).permutation(E)
    bias = np.empty(E, np.float64)
    bias[perm] = np.log(p)
    return bias.astype(np.float32)
