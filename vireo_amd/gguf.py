"""GGUF files for the MoE path.

* GGUFWriter: writes GGUF v3 files (metadata of every scalar type, strings,
  arrays, tensors at the file's alignment).
* write_moe_gguf: a synthetic MoE model file with the tensor names and
  metadata keys of a real MoE GGUF (src/gguf_run.c:276-318): per layer
  blk.<l>.ffn_gate_inp (F32 router), ffn_gate_exps / ffn_up_exps /
  ffn_down_exps (stacked experts, expert-major) and ffn_norm, plus
  token_embd, output_norm and optionally an untied output head; weights are
  the deterministic synthetic weights of vireo_amd.workloads.
* GGUFModel: the device model that vireo_gguf_moe_load builds from a file
  (routers, norms and head in HBM, experts paged by the ExpertStore).
"""
import ctypes as C
import struct

import numpy as np

from . import _lib
from . import workloads as W

# metadata value types (src/gguf.h:16-18)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype, value, arr_type=None):
    """Encoded value; for an ARRAY, arr_type is the item type, or a tuple
    (ARRAY, item type of the inner arrays) for an array of arrays."""
    if vtype == STRING:
        return _str(value)
    if vtype == ARRAY:
        item, inner = arr_type if isinstance(arr_type, tuple) else (arr_type, None)
        out = struct.pack("<IQ", item, len(value))
        return out + b"".join(_value(item, v, inner) for v in value)
    return struct.pack(_FMT[vtype], value)


class GGUFWriter:
    """Collects metadata and tensors, then writes one GGUF v3 file."""

    def __init__(self, alignment=32):
        self.alignment = alignment
        self.kv = []
        self.tensors = []
        if alignment != 32:
            self.add("general.alignment", U32, alignment)

    def add(self, key, vtype, value, arr_type=None):
        self.kv.append((key, vtype, value, arr_type))

    def add_tensor(self, name, dims, ggml_type, data):
        """dims in GGUF order: dims[0] is the row length."""
        self.tensors.append((name, list(dims), ggml_type, np.ascontiguousarray(data).view(np.uint8).reshape(-1)))

    def write(self, path, progress=None):
        """progress (optional): called with a message every 64 tensors written."""
        a = self.alignment
        head = [b"GGUF", struct.pack("<IQQ", 3, len(self.tensors), len(self.kv))]
        for key, vtype, value, arr_type in self.kv:
            head.append(_str(key) + struct.pack("<I", vtype) + _value(vtype, value, arr_type))
        offsets, off = [], 0
        for _, _, _, data in self.tensors:
            offsets.append(off)
            off += (len(data) + a - 1) // a * a
        for (name, dims, typ, _), o in zip(self.tensors, offsets):
            head.append(_str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims) +
                        struct.pack("<IQ", typ, o))
        blob = b"".join(head)
        with open(path, "wb") as f:
            f.write(blob)
            f.write(b"\0" * ((a - len(blob) % a) % a))
            for i, ((_, _, _, data), o) in enumerate(zip(self.tensors, offsets)):
                f.write(memoryview(data))
                f.write(b"\0" * ((a - len(data) % a) % a))
                if progress and i % 64 == 63:
                    progress(f"{i + 1} of {len(self.tensors)} tensors written")


def moe_arch(shape):
    """Architecture name whose loader rule gives the shape's renormalisation
    (src/gguf_run.c:292: every architecture but "olmoe" renormalises)."""
    return "qwen3moe" if shape.renorm else "olmoe"


def write_moe_gguf(path, shape, n_layers, seed, vocab=0, untied=False, norms=True, alignment=32, arch=None,
                   lm_type=W.Q8_0, progress=None, layer_bytes=None):
    """Write a synthetic MoE GGUF file; returns the host arrays written, for
    checking (routers [L][E x d], experts [L] (gate_all, up_all, down_all),
    ffn_norm [L][d] or None, and with vocab: out_norm, token_embd, output).
    progress (optional): called with a message as layers are made and written.
    layer_bytes (optional): layer -> (gate_all, up_all, down_all), the same
    bytes as workloads.host_layer (e.g. copied from a device-made layer)."""
    d, E, fe = shape.d, shape.E, shape.fe
    arch = arch or moe_arch(shape)
    w = GGUFWriter(alignment)
    w.add("general.architecture", STRING, arch)
    w.add("general.name", STRING, f"synthetic {shape.name}")
    w.add(f"{arch}.block_count", U32, n_layers)
    w.add(f"{arch}.embedding_length", U32, d)
    w.add(f"{arch}.feed_forward_length", U32, 4 * d)
    w.add(f"{arch}.expert_feed_forward_length", U32, fe)
    w.add(f"{arch}.expert_count", U32, E)
    w.add(f"{arch}.expert_used_count", U32, shape.k)
    w.add(f"{arch}.attention.layer_norm_rms_epsilon", F32, W.EPS)
    if vocab:
        w.add("tokenizer.ggml.tokens", ARRAY, [f"<t{i}>" for i in range(vocab)], STRING)
        w.add("tokenizer.ggml.scores", ARRAY, [float(-i) for i in range(vocab)], F32)
    out = {"routers": [], "experts": [], "ffn_norm": [] if norms else None}
    for l in range(n_layers):
        r = W.host_router(shape, l, seed)
        g, u, dn = layer_bytes(l) if layer_bytes else W.host_layer(shape, l, seed)
        w.add_tensor(f"blk.{l}.ffn_gate_inp.weight", [d, E], W.F32, r)
        w.add_tensor(f"blk.{l}.ffn_gate_exps.weight", [d, fe, E], shape.gate_type, g)
        w.add_tensor(f"blk.{l}.ffn_up_exps.weight", [d, fe, E], shape.up_type, u)
        w.add_tensor(f"blk.{l}.ffn_down_exps.weight", [fe, d, E], shape.down_type, dn)
        out["routers"].append(r)
        out["experts"].append((g, u, dn))
        if progress and l % 8 == 7:
            progress(f"{l + 1} of {n_layers} layers made")
        if norms:
            nw = (1.0 + 0.25 * W.host_normal(d, seed, W.stream_id(l, 15))).astype(np.float32)
            w.add_tensor(f"blk.{l}.ffn_norm.weight", [d], W.F32, nw)
            out["ffn_norm"].append(nw)
    if vocab:
        emb = W.host_matrix(lm_type, d, 0, vocab, seed, W.stream_id(0, W.KIND_LM_HEAD))
        on = (1.0 + 0.25 * W.host_normal(d, seed, W.stream_id(n_layers, 15))).astype(np.float32)
        w.add_tensor("token_embd.weight", [d, vocab], lm_type, emb)
        w.add_tensor("output_norm.weight", [d], W.F32, on)
        out["token_embd"], out["out_norm"], out["output"] = emb, on, emb
        if untied:
            head = W.host_matrix(lm_type, d, 0, vocab, seed + 1, W.stream_id(0, W.KIND_LM_HEAD))
            w.add_tensor("output.weight", [d, vocab], lm_type, head)
            out["output"] = head
    w.write(path, progress)
    return out


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


class GGUFModel:
    """vireo_gguf_moe_load: an MoE GGUF file on the device."""

    def __init__(self, path, expert_capacity=0, load_head=True):
        self.lib = _lib.load()
        p = C.POINTER(_lib.GGUFMoE)()
        rc = self.lib.vireo_gguf_moe_load(str(path).encode(), expert_capacity, int(load_head), C.byref(p))
        if rc:
            why = self.lib.vireo_gguf_moe_error()
            raise _lib.VireoError(f"vireo_gguf_moe_load({path}) failed: {rc} ({why.decode() if why else '?'})")
        self.p = p
        m = p.contents
        self.arch = m.arch.decode()
        self.vocab, self.eps = m.vocab, m.eps
        md = m.model
        self.d, self.E, self.k, self.fe = md.dim, md.n_experts, md.n_used, md.ffn_exp
        self.renorm, self.n_layers = bool(md.topk_renorm), md.n_layers

    def forward(self, layer, x, hb, stream=None, return_routing=False):
        """x[t] += moe(hb[t]) in place (moe_ffn_forward)."""
        import torch
        T = hb.shape[0]
        idx = w = None
        if return_routing:
            idx = torch.empty((T, self.k), dtype=torch.int32, device=hb.device)
            w = torch.empty((T, self.k), dtype=torch.float32, device=hb.device)
        _lib.check(self.lib.moe_ffn_forward(C.byref(self.p.contents.model), layer, _ptr(x), _ptr(hb), T, _ptr(idx),
                                            _ptr(w), _stream(stream)), "moe_ffn_forward")
        return (idx, w) if return_routing else None

    def step(self, token, x, xb, logits, stream=None):
        """moe_stack_step on the file's norms and head."""
        _lib.check(self.lib.moe_stack_step(C.byref(self.p.contents.stack), _ptr(token), _ptr(x), _ptr(xb),
                                           _ptr(logits), _stream(stream)), "moe_stack_step")

    def stats(self):
        """The reference's ExpertStats for the work done so far (expert_store_stats)."""
        st = _lib.ExpertStats()
        self.lib.expert_store_stats(self.p.contents.model.es, C.byref(st))
        return {n: getattr(st, n) for n, _ in _lib.ExpertStats._fields_}

    def hbm_stats(self):
        """What the HBM pool did (expert_store_hbm_stats; resident_bytes
        includes the packed copies of pinned layers)."""
        st = _lib.ExpertStats()
        self.lib.expert_store_hbm_stats(self.p.contents.model.es, C.byref(st))
        return {n: getattr(st, n) for n, _ in _lib.ExpertStats._fields_}

    def packed_bytes(self):
        """Bytes of the kernels' packed copies of pinned layers (expert_store_packed_bytes)."""
        return int(self.lib.expert_store_packed_bytes(self.p.contents.model.es))

    def set_prefetch(self, on):
        """Let paged calls read guessed next-layer experts ahead (expert_store_set_prefetch)."""
        _lib.check(self.lib.expert_store_set_prefetch(self.p.contents.model.es, int(bool(on))),
                   "expert_store_set_prefetch")

    def prefetch_stats(self):
        """Experts read ahead, those of them looked up before eviction, bytes read ahead."""
        out = (C.c_uint64 * 3)()
        self.lib.expert_store_prefetch_stats(self.p.contents.model.es, out)
        return {"issued": out[0], "used": out[1], "bytes": out[2]}

    def close(self):
        if getattr(self, "p", None):
            self.lib.vireo_gguf_moe_free(self.p)
            self.p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# stream kinds of the attention and dense-FFN tensors (after the MoE kinds
# of vireo_amd.workloads; 15 is the norms')
KIND_WQ, KIND_WK, KIND_WV, KIND_WO, KIND_FG, KIND_FU, KIND_FD, KIND_VEC = range(7, 15)


def write_model_gguf(path, arch, n_layers, d, n_heads, n_kv_heads, head_size, vocab, seed, attn_type=W.Q8_0,
                     moe=None, ffn=0, ffn_types=(W.Q4_K, W.Q4_K, W.Q6_K), bias=False, qk_norm="head",
                     norm_type=W.F32, untied=False, rope_base=1000000.0, lm_type=W.Q8_0, explicit_head=True):
    """Write a synthetic whole-model GGUF file with the tensor names and
    metadata keys the reference's loader reads (src/gguf_run.c:276-318):
    per block attn_norm, attn_q/k/v (+ .bias with `bias`), attn_q_norm /
    attn_k_norm (qk_norm "head": [head_size], "full": [heads * head_size],
    None: absent), attn_output, ffn_norm, and either the MoE tensors of
    `moe` (a workloads.MoEShape with d == moe.d) or a dense SwiGLU FFN of
    width ffn with types ffn_types; token_embd, output_norm and, with
    untied, output. Norm weights are 1 + 0.25 N(0, 1) stored as norm_type,
    biases N(0, 0.1). Returns the file's expert shape (or None)."""
    w = GGUFWriter()
    w.add("general.architecture", STRING, arch)
    w.add("general.name", STRING, "synthetic whole model")
    w.add(f"{arch}.block_count", U32, n_layers)
    w.add(f"{arch}.embedding_length", U32, d)
    w.add(f"{arch}.feed_forward_length", U32, ffn if ffn else 4 * d)
    w.add(f"{arch}.attention.head_count", U32, n_heads)
    w.add(f"{arch}.attention.head_count_kv", U32, n_kv_heads)
    if explicit_head:
        w.add(f"{arch}.attention.key_length", U32, head_size)
    else:
        assert head_size == d // n_heads
    w.add(f"{arch}.attention.layer_norm_rms_epsilon", F32, W.EPS)
    w.add(f"{arch}.rope.freq_base", F32, rope_base)
    if moe is not None:
        assert moe.d == d
        w.add(f"{arch}.expert_feed_forward_length", U32, moe.fe)
        w.add(f"{arch}.expert_count", U32, moe.E)
        w.add(f"{arch}.expert_used_count", U32, moe.k)
        w.add(f"{arch}.expert_weights_norm", U32, int(moe.renorm))
    nq, nk = n_heads * head_size, n_kv_heads * head_size

    def vec(n, l, slot, base, sigma):
        v = (base + sigma * W.host_normal(n, seed, W.stream_id(l, KIND_VEC), first=slot * 65536)).astype(np.float32)
        if norm_type == W.F16:
            return [n], W.F16, v.astype(np.float16)
        return [n], W.F32, v

    def mat(name, typ, cols, rows, l, kind, sigma=W.WEIGHT_SIGMA):
        w.add_tensor(name, [cols, rows], typ, W.host_matrix(typ, cols, 0, rows, seed, W.stream_id(l, kind), sigma))

    for l in range(n_layers):
        w.add_tensor(f"blk.{l}.attn_norm.weight", *vec(d, l, 0, 1.0, 0.25))
        mat(f"blk.{l}.attn_q.weight", attn_type, d, nq, l, KIND_WQ, 0.05)
        mat(f"blk.{l}.attn_k.weight", attn_type, d, nk, l, KIND_WK, 0.05)
        mat(f"blk.{l}.attn_v.weight", attn_type, d, nk, l, KIND_WV, 0.05)
        mat(f"blk.{l}.attn_output.weight", attn_type, nq, d, l, KIND_WO, 0.05)
        if bias:
            w.add_tensor(f"blk.{l}.attn_q.bias", *vec(nq, l, 1, 0.0, 0.1))
            w.add_tensor(f"blk.{l}.attn_k.bias", *vec(nk, l, 2, 0.0, 0.1))
            w.add_tensor(f"blk.{l}.attn_v.bias", *vec(nk, l, 3, 0.0, 0.1))
        if qk_norm:
            w.add_tensor(f"blk.{l}.attn_q_norm.weight", *vec(head_size if qk_norm == "head" else nq, l, 4, 1.0, 0.25))
            w.add_tensor(f"blk.{l}.attn_k_norm.weight", *vec(head_size if qk_norm == "head" else nk, l, 5, 1.0, 0.25))
        w.add_tensor(f"blk.{l}.ffn_norm.weight", *vec(d, l, 6, 1.0, 0.25))
        if moe is not None:
            E, fe = moe.E, moe.fe
            g, u, dn = W.host_layer(moe, l, seed)
            w.add_tensor(f"blk.{l}.ffn_gate_inp.weight", [d, E], W.F32, W.host_router(moe, l, seed))
            w.add_tensor(f"blk.{l}.ffn_gate_exps.weight", [d, fe, E], moe.gate_type, g)
            w.add_tensor(f"blk.{l}.ffn_up_exps.weight", [d, fe, E], moe.up_type, u)
            w.add_tensor(f"blk.{l}.ffn_down_exps.weight", [fe, d, E], moe.down_type, dn)
        else:
            mat(f"blk.{l}.ffn_gate.weight", ffn_types[0], d, ffn, l, KIND_FG)
            mat(f"blk.{l}.ffn_up.weight", ffn_types[1], d, ffn, l, KIND_FU)
            mat(f"blk.{l}.ffn_down.weight", ffn_types[2], ffn, d, l, KIND_FD)
    emb = W.host_matrix(lm_type, d, 0, vocab, seed, W.stream_id(0, W.KIND_LM_HEAD), 0.5)
    w.add_tensor("token_embd.weight", [d, vocab], lm_type, emb)
    w.add_tensor("output_norm.weight", *vec(d, n_layers, 7, 1.0, 0.25))
    if untied:
        w.add_tensor("output.weight", [d, vocab], lm_type,
                     W.host_matrix(lm_type, d, 0, vocab, seed + 1, W.stream_id(0, W.KIND_LM_HEAD)))
    w.write(path)
    return moe
