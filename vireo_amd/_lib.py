"""ctypes bindings for libvireo_hip.so (the C-ABI declared in include/*.h).

The library is built in-tree by vireo_amd.build; loading fails loudly when it
is missing, because there is no CPU fallback for any of these entry points.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvireo_hip.so")

c_vp = C.c_void_p
c_i32p = C.POINTER(C.c_int32)


class GGUFStr(C.Structure):
    """gguf_str: `len` bytes at `ptr` (inside a file mapping: not NUL-terminated)."""
    _fields_ = [("ptr", c_vp), ("len", C.c_uint64)]

    def text(self):
        return C.string_at(self.ptr, self.len).decode("utf-8", "replace") if self.len else ""


class GGUFTensor(C.Structure):
    """gguf_tensor (src/gguf.h:36-45); only data and ggml_type are read."""
    _fields_ = [
        ("name", GGUFStr),
        ("n_dims", C.c_uint32),
        ("dims", C.c_uint64 * 4),
        ("ggml_type", C.c_uint32),
        ("offset", C.c_uint64),
        ("data", c_vp),
        ("n_elems", C.c_uint64),
        ("nbytes", C.c_uint64),
    ]


class ExpertStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "requests", "hits", "misses", "bytes_read", "resident_bytes", "capacity_bytes", "experts_resident")]


class ExpertSlices(C.Structure):
    _fields_ = [
        ("gate_off", C.c_uint64), ("up_off", C.c_uint64), ("down_off", C.c_uint64),
        ("gate_bytes", C.c_uint32), ("up_bytes", C.c_uint32), ("down_bytes", C.c_uint32),
    ]


class ExpertView(C.Structure):
    _fields_ = [("gate", c_vp), ("up", c_vp), ("down", c_vp), ("slot", c_vp)]


class MoELayer(C.Structure):
    _fields_ = [
        ("router", C.POINTER(GGUFTensor)),
        ("gate_exps", C.POINTER(GGUFTensor)),
        ("up_exps", C.POINTER(GGUFTensor)),
        ("down_exps", C.POINTER(GGUFTensor)),
        ("logit_bias", c_vp),
    ]


class MoEModel(C.Structure):
    _fields_ = [
        ("dim", C.c_int), ("n_experts", C.c_int), ("n_used", C.c_int), ("ffn_exp", C.c_int),
        ("topk_renorm", C.c_int), ("n_layers", C.c_int),
        ("layers", C.POINTER(MoELayer)),
        ("es", c_vp),
    ]


class MoEStack(C.Structure):
    _fields_ = [
        ("moe", C.POINTER(MoEModel)),
        ("ffn_norm", c_vp),
        ("out_norm", c_vp),
        ("lm_head", C.POINTER(GGUFTensor)),
        ("vocab", C.c_int),
        ("eps", C.c_float),
        ("tok_embd", C.POINTER(GGUFTensor)),
    ]


class GGUFKV(C.Structure):
    """gguf_kv (src/gguf.h:27-34); `val` is the union's 8 bytes."""
    _fields_ = [
        ("key", GGUFStr),
        ("type", C.c_uint32),
        ("val", C.c_uint64),
        ("str", GGUFStr),
        ("arr_type", C.c_uint32),
        ("arr_len", C.c_uint64),
        ("arr_data", c_vp),
    ]


class GGUFCtx(C.Structure):
    """gguf_ctx (src/gguf.h:47-55)."""
    _fields_ = [
        ("fd", C.c_int), ("map", c_vp), ("size", C.c_size_t),
        ("version", C.c_uint32),
        ("n_tensors", C.c_uint64), ("n_kv", C.c_uint64),
        ("kv", C.POINTER(GGUFKV)),
        ("tensors", C.POINTER(GGUFTensor)),
        ("data", c_vp),
        ("alignment", C.c_uint64),
    ]


class GGUFMoE(C.Structure):
    """vireo_gguf_moe (include/vireo_hip.h)."""
    _fields_ = [
        ("gguf", C.POINTER(GGUFCtx)),
        ("arch", C.c_char * 64),
        ("model", MoEModel),
        ("stack", MoEStack),
        ("vocab", C.c_int),
        ("eps", C.c_float),
        ("priv", c_vp),
    ]


class KVConfig(C.Structure):
    """VireoKVConfig: the layout of KVConfig (src/kvstore.h:26-33)."""
    _fields_ = [("n_layers", C.c_int), ("kv_dim", C.c_int), ("block_tokens", C.c_int), ("sink_tokens", C.c_int),
                ("window_tokens", C.c_int), ("capacity_bytes", C.c_uint64)]


class KVStats(C.Structure):
    """VireoKVStats: the layout of KVStats (src/kvstore.h:35-44)."""
    _fields_ = [(n, C.c_uint64) for n in ("requests", "hits", "misses", "prefetched", "bytes_read", "bytes_spilled",
                                          "resident_bytes", "capacity_bytes")]


class Block(C.Structure):
    """vireo_block (include/vireo_hip.h): one transformer block's device tensors."""
    _fields_ = [
        ("attn_norm", c_vp),
        ("wq", C.POINTER(GGUFTensor)), ("wk", C.POINTER(GGUFTensor)), ("wv", C.POINTER(GGUFTensor)),
        ("bq", c_vp), ("bk", c_vp), ("bv", c_vp),
        ("q_norm", c_vp), ("k_norm", c_vp),
        ("q_norm_len", C.c_int), ("k_norm_len", C.c_int),
        ("wo", C.POINTER(GGUFTensor)),
        ("ffn_norm", c_vp),
        ("wg", C.POINTER(GGUFTensor)), ("wu", C.POINTER(GGUFTensor)), ("wd", C.POINTER(GGUFTensor)),
    ]


class Model(C.Structure):
    """vireo_model (include/vireo_hip.h)."""
    _fields_ = [
        ("n_layers", C.c_int), ("dim", C.c_int), ("n_heads", C.c_int), ("n_kv_heads", C.c_int),
        ("head_size", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int),
        ("eps", C.c_float), ("rope_base", C.c_float),
        ("blocks", C.POINTER(Block)),
        ("moe", C.POINTER(MoEModel)),
        ("tok_embd", C.POINTER(GGUFTensor)),
        ("out_norm", c_vp),
        ("lm_head", C.POINTER(GGUFTensor)),
        ("rope", c_vp),
        ("max_pos", C.c_int),
    ]


class GGUFModelC(C.Structure):
    """vireo_gguf_model (include/vireo_hip.h)."""
    _fields_ = [
        ("gguf", C.POINTER(GGUFCtx)),
        ("arch", C.c_char * 64),
        ("model", Model),
        ("moe", MoEModel),
        ("priv", c_vp),
    ]


# name -> (restype, argtypes)
SIGNATURES = {
    "vireo_hip_init": (C.c_int, [C.c_int]),
    "vireo_hip_strerror": (C.c_char_p, [C.c_int]),
    "vireo_type_block": (C.c_int, [C.c_uint32, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "qmatvec": (C.c_int, [c_vp, c_vp, C.POINTER(GGUFTensor), C.c_int, C.c_int]),
    "qmatvec_async": (C.c_int, [c_vp, c_vp, C.POINTER(GGUFTensor), C.c_int, C.c_int, c_vp]),
    "qdequant_rows": (C.c_int, [C.c_uint32, c_vp, c_vp, C.c_int, C.c_int, c_vp]),
    "vireo_rmsnorm": (C.c_int, [c_vp, c_vp, c_vp, C.c_int, C.c_int, C.c_float, c_vp]),
    "vireo_router_logits": (C.c_int, [c_vp, c_vp, C.c_int, C.c_int, C.c_int, c_vp, c_vp]),
    "vireo_argmax": (C.c_int, [c_vp, C.c_int, c_vp, c_vp]),
    "vireo_embed": (C.c_int, [C.c_uint32, c_vp, C.c_int, C.c_int, c_vp, C.c_int, c_vp, c_vp]),
    "moe_stack_step": (C.c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "moe_stack_step_trace": (C.c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "moe_route": (C.c_int, [C.POINTER(MoEModel), C.c_int, c_vp, C.c_int, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "moe_dispatch": (C.c_int, [c_vp, C.c_int, C.c_int, C.c_int, c_vp, c_vp, c_vp, c_vp]),
    "vireo_hip_set_path": (C.c_int, [C.c_int]),
    "vireo_hip_set_packed": (C.c_int, [C.c_int]),
    "moe_decode_state_bytes": (C.c_int64, [C.POINTER(MoEModel)]),
    "moe_decode_stage": (C.c_int, [C.POINTER(MoEModel), C.c_int, C.c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "moe_decode_stage_timed": (C.c_int, [C.POINTER(MoEModel), C.c_int, C.c_int, c_vp, c_vp, c_vp, c_vp, C.c_int64,
                                         c_vp, c_vp, c_vp, c_vp]),
    "moe_decode_phases": (C.c_int, [C.POINTER(MoEModel), C.c_int, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "moe_ffn_forward": (C.c_int, [C.POINTER(MoEModel), C.c_int, c_vp, c_vp, C.c_int, c_vp, c_vp, c_vp]),
    "moe_ffn_forward_noalloc": (C.c_int, [C.POINTER(MoEModel), C.c_int, c_vp, c_vp, C.c_int, c_vp, c_vp, c_vp]),
    "expert_store_create": (c_vp, [C.c_int, C.c_uint64, C.c_int, C.c_int]),
    "expert_store_create_device": (c_vp, [c_vp, C.c_uint64, C.c_uint64, C.c_int, C.c_int]),
    "expert_store_register": (None, [c_vp, C.c_int, C.c_int, C.POINTER(ExpertSlices)]),
    "expert_store_lookup": (C.c_int, [c_vp, C.c_int, C.c_int, C.POINTER(ExpertView)]),
    "expert_store_release": (None, [c_vp, C.POINTER(ExpertView)]),
    "expert_store_stats": (None, [c_vp, C.POINTER(ExpertStats)]),
    "expert_store_hbm_stats": (None, [c_vp, C.POINTER(ExpertStats)]),
    "expert_store_packed_bytes": (C.c_uint64, [c_vp]),
    "vireo_rmsnorm_exact": (C.c_int, [c_vp, c_vp, c_vp, C.c_int, C.c_float, c_vp]),
    "expert_store_set_prefetch": (C.c_int, [c_vp, C.c_int]),
    "expert_store_prefetch_stats": (None, [c_vp, C.POINTER(C.c_uint64)]),
    "vireo_hip_status": (C.c_int, [c_vp]),
    "vireo_hip_set_spin_limit": (C.c_int, [C.c_uint]),
    "expert_store_destroy": (None, [c_vp]),
    "expert_store_pin_layer": (C.c_int, [c_vp, C.c_int, C.POINTER(c_vp)]),
    "expert_store_unpin_layer": (C.c_int, [c_vp, C.c_int]),
    "vireo_synth_normal": (C.c_int, [c_vp, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float]),
    "vireo_quantize": (C.c_int, [C.c_uint32, c_vp, c_vp, C.c_int, C.c_int64]),
    "vireo_synth_matrix": (C.c_int, [C.c_uint32, c_vp, C.c_int, C.c_int64, C.c_int64, C.c_uint64, C.c_uint64,
                                     C.c_float]),
    "vireo_synth_matrix_dev": (C.c_int, [C.c_uint32, c_vp, C.c_int, C.c_int64, C.c_int64, C.c_uint64, C.c_uint64,
                                         C.c_float, c_vp]),
    "vireo_synth_hidden": (C.c_int, [c_vp, c_vp, C.c_int, C.c_int64, C.c_uint64, C.c_uint64, C.c_float]),
    "vireo_row_bytes": (C.c_int64, [C.c_uint32, C.c_int]),
    "vireo_gguf_open": (C.POINTER(GGUFCtx), [C.c_char_p]),
    "vireo_gguf_close": (None, [C.POINTER(GGUFCtx)]),
    "vireo_gguf_find": (C.POINTER(GGUFKV), [C.POINTER(GGUFCtx), C.c_char_p]),
    "vireo_gguf_get_u64": (C.c_int, [C.POINTER(GGUFCtx), C.c_char_p, C.POINTER(C.c_uint64)]),
    "vireo_gguf_get_f32": (C.c_int, [C.POINTER(GGUFCtx), C.c_char_p, C.POINTER(C.c_float)]),
    "vireo_gguf_get_str": (c_vp, [C.POINTER(GGUFCtx), C.c_char_p, C.POINTER(C.c_uint64)]),
    "vireo_gguf_tensor_by_name": (C.POINTER(GGUFTensor), [C.POINTER(GGUFCtx), C.c_char_p]),
    "vireo_gguf_moe_load": (C.c_int, [C.c_char_p, C.c_uint64, C.c_int, C.POINTER(C.POINTER(GGUFMoE))]),
    "vireo_gguf_moe_error": (C.c_char_p, []),
    "vireo_gguf_moe_free": (None, [C.POINTER(GGUFMoE)]),
    "vireo_rope_table": (C.c_int, [C.c_float, C.c_int, C.c_int, c_vp]),
    "vireo_model_state_bytes": (C.c_int64, [C.POINTER(Model)]),
    "vireo_model_step": (C.c_int, [C.POINTER(Model), c_vp, c_vp, C.c_int, C.c_int, c_vp, c_vp, c_vp, c_vp]),
    "vireo_model_step_pos": (C.c_int, [C.POINTER(Model), c_vp, c_vp, c_vp, C.c_int, c_vp, c_vp, c_vp, c_vp]),
    "vireo_kv_create_contiguous": (c_vp, [KVConfig, C.c_int]),
    "vireo_kv_append_pos": (C.c_int, [c_vp, C.c_int, C.c_int, c_vp, c_vp, c_vp, c_vp]),
    "vireo_kv_attend_gqa_pos": (C.c_int, [c_vp, C.c_int, C.c_int, C.c_int, c_vp, c_vp, c_vp, c_vp]),
    "vireo_gguf_model_load": (C.c_int, [C.c_char_p, C.c_uint64, C.c_int, C.POINTER(C.POINTER(GGUFModelC))]),
    "vireo_gguf_model_free": (None, [C.POINTER(GGUFModelC)]),
    "vireo_kv_create_dense": (c_vp, [KVConfig]),
    "vireo_kv_create_paged": (c_vp, [KVConfig, C.c_int, C.c_int]),
    "vireo_kv_append": (C.c_int, [c_vp, C.c_int, C.c_int, c_vp, c_vp, c_vp]),
    "vireo_kv_append_n": (C.c_int, [c_vp, C.c_int, C.c_int, C.c_int, c_vp, c_vp, c_vp]),
    "vireo_kv_attend": (C.c_int, [c_vp, C.c_int, c_vp, c_vp, c_vp]),
    "vireo_kv_attend_gqa": (C.c_int, [c_vp, C.c_int, C.c_int, C.c_int, c_vp, c_vp, c_vp]),
    "vireo_kv_stats": (None, [c_vp, C.POINTER(KVStats)]),
    "vireo_kv_destroy": (None, [c_vp]),
}

_lib = None


class VireoError(RuntimeError):
    pass


def load():
    """Load libvireo_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise VireoError(f"{LIB_PATH} is missing: run `python -m vireo_amd.build` (no CPU fallback exists)")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc, what="vireo-hip call"):
    if rc != 0:
        msg = load().vireo_hip_strerror(rc)
        raise VireoError(f"{what} failed: {rc} ({msg.decode() if msg else '?'})")
    return rc
