"""The GPU KV store (include/vireo_kv.h) from Python: DeviceKV wraps
vireo_kv_create_dense / vireo_kv_create_paged and their operations on torch
device tensors."""
import ctypes as C

from . import _lib

ALL, RECENT, TOPK = 0, 1, 2


def _ptr(t):
    return C.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


class DeviceKV:
    """KV cache of n_layers (layer x kv-head) rows of kv_dim floats.
    dense=True: the reference's dense store; else its out-of-core store with
    `strategy` (ALL, RECENT, TOPK with topk_budget) over capacity_bytes of HBM."""

    def __init__(self, n_layers, kv_dim, block_tokens, sink_tokens=0, window_tokens=0, capacity_bytes=0,
                 dense=False, strategy=ALL, topk_budget=0, max_tokens=0):
        """max_tokens > 0: a contiguous dense store (vireo_kv_create_contiguous)
        that also takes device positions (append_pos / attend_gqa_pos)."""
        self.lib = _lib.load()
        cfg = _lib.KVConfig(n_layers, kv_dim, block_tokens, sink_tokens, window_tokens, capacity_bytes)
        if max_tokens > 0:
            self.h = self.lib.vireo_kv_create_contiguous(cfg, max_tokens)
        else:
            self.h = (self.lib.vireo_kv_create_dense(cfg) if dense
                      else self.lib.vireo_kv_create_paged(cfg, strategy, topk_budget))
        if not self.h:
            raise _lib.VireoError("vireo_kv_create failed (check kv_dim in {64, 128, 256}, block_tokens <= 64)")
        self.kv_dim = kv_dim

    def append(self, layer, pos, k, v, stream=None):
        """k, v: [kv_dim] or [n, kv_dim] (rows for layers layer .. layer + n - 1)."""
        n = 1 if k.dim() == 1 else k.shape[0]
        _lib.check(self.lib.vireo_kv_append_n(self.h, layer, n, pos, _ptr(k), _ptr(v), _stream(stream)),
                   "vireo_kv_append_n")

    def append_pos(self, layer, pos, k, v, stream=None):
        """append at the device position pos (int32 tensor [1])."""
        n = 1 if k.dim() == 1 else k.shape[0]
        _lib.check(self.lib.vireo_kv_append_pos(self.h, layer, n, _ptr(pos), _ptr(k), _ptr(v), _stream(stream)),
                   "vireo_kv_append_pos")

    def attend_gqa_pos(self, layer0, n_heads, n_kv_heads, pos, q, out, stream=None):
        _lib.check(self.lib.vireo_kv_attend_gqa_pos(self.h, layer0, n_heads, n_kv_heads, _ptr(pos), _ptr(q), _ptr(out),
                                                    _stream(stream)), "vireo_kv_attend_gqa_pos")

    def attend(self, layer, q, out, stream=None):
        _lib.check(self.lib.vireo_kv_attend(self.h, layer, _ptr(q), _ptr(out), _stream(stream)), "vireo_kv_attend")

    def attend_gqa(self, layer0, n_heads, n_kv_heads, q, out, stream=None):
        _lib.check(self.lib.vireo_kv_attend_gqa(self.h, layer0, n_heads, n_kv_heads, _ptr(q), _ptr(out),
                                                _stream(stream)), "vireo_kv_attend_gqa")

    def stats(self):
        st = _lib.KVStats()
        self.lib.vireo_kv_stats(self.h, C.byref(st))
        return {n: getattr(st, n) for n, _ in _lib.KVStats._fields_}

    def close(self):
        if getattr(self, "h", None):
            self.lib.vireo_kv_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
