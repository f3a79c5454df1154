"""Whole-model decode on the device: vireo_gguf_model_load + vireo_model_step
(include/vireo_hip.h), the reference's forward() (src/gguf_run.c:216-251)
over a GGUF file with a dense GPU KV store."""
import ctypes as C

from . import _lib
from .kv import DeviceKV


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


class GGUFDecoder:
    """A GGUF model on the device with its KV store (block_tokens per block,
    the reference runner's default sink and window): step(token, pos) runs
    one forward() and, with want_logits, returns the greedy next token."""

    def __init__(self, path, max_pos=256, expert_capacity=0, block_tokens=32, device="cuda", contiguous=False):
        import torch
        self.lib = _lib.load()
        p = C.POINTER(_lib.GGUFModelC)()
        rc = self.lib.vireo_gguf_model_load(str(path).encode(), expert_capacity, max_pos, C.byref(p))
        if rc:
            why = self.lib.vireo_gguf_moe_error()
            raise _lib.VireoError(f"vireo_gguf_model_load({path}) failed: {rc} ({why.decode() if why else '?'})")
        self.p = p
        m = p.contents.model
        self.arch = p.contents.arch.decode()
        self.dim, self.vocab, self.n_layers = m.dim, m.vocab, m.n_layers
        self.n_heads, self.n_kv_heads, self.head_size = m.n_heads, m.n_kv_heads, m.head_size
        self.is_moe = bool(m.moe)
        self.kv = DeviceKV(self.n_layers * self.n_kv_heads, self.head_size, block_tokens, 32, 256, dense=True,
                           max_tokens=max_pos if contiguous else 0)
        self.pos = torch.zeros(1, dtype=torch.int32, device=device)
        nbytes = self.lib.vireo_model_state_bytes(C.byref(m))
        if nbytes < 0:
            raise _lib.VireoError(f"vireo_model_state_bytes failed: {nbytes}")
        self.state = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)
        self.x = torch.empty(self.dim, dtype=torch.float32, device=device)
        self.logits = torch.empty(self.vocab, dtype=torch.float32, device=device)
        self.token = torch.zeros(1, dtype=torch.int32, device=device)

    def step(self, token, pos, want_logits=True, stream=None):
        """forward(token, pos); returns argmax(logits) (as int) with want_logits, else None."""
        self.token.fill_(int(token))
        _lib.check(self.lib.vireo_model_step(C.byref(self.p.contents.model), C.c_void_p(self.kv.h), _ptr(self.token),
                                             pos, int(want_logits), _ptr(self.x),
                                             _ptr(self.logits) if want_logits else None, _ptr(self.state),
                                             _stream(stream)), "vireo_model_step")
        return int(self.token.item()) if want_logits else None

    def step_pos(self, want_logits=True, stream=None):
        """vireo_model_step_pos: forward(self.token, self.pos) with both on the
        device; self.token receives the greedy token, self.pos advances."""
        _lib.check(self.lib.vireo_model_step_pos(C.byref(self.p.contents.model), C.c_void_p(self.kv.h),
                                                 _ptr(self.token), _ptr(self.pos), int(want_logits), _ptr(self.x),
                                                 _ptr(self.logits) if want_logits else None, _ptr(self.state),
                                                 _stream(stream)), "vireo_model_step_pos")

    def close(self):
        if getattr(self, "kv", None):
            self.kv.close()
            self.kv = None
        if getattr(self, "p", None):
            self.lib.vireo_gguf_model_free(self.p)
            self.p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceModel:
    """A synthetic whole model on the device for measurement: every block has
    grouped-query attention (q/k/v/output matrices generated on the GPU in the
    given types, unit per-head QK-norm weights) and the MoE FFN of a
    stack.DeviceStack, whose Q8_0 LM head is also the token embedding (tied);
    norm weights are unit weights. KV store: dense, block_tokens per block."""

    def __init__(self, shape, n_layers, n_heads=32, n_kv_heads=4, head_size=128, vocab=None, max_pos=8192,
                 seed=1234, attn_types=None, block_tokens=32, rope_base=1000000.0, device="cuda", contiguous=False):
        import torch
        from . import stack as S
        from . import workloads as W
        from . import moe as M
        from .gguf import KIND_WQ
        self.lib = _lib.load()
        vocab = vocab or W.LM_VOCAB
        attn_types = attn_types or (W.Q4_K, W.Q4_K, W.Q6_K, W.Q4_K)
        self.stack = S.DeviceStack(shape, n_layers, vocab=vocab, seed=seed, device=device)
        d, nq, nk = shape.d, n_heads * head_size, n_kv_heads * head_size
        dims = [(d, nq), (d, nk), (d, nk), (nq, d)]  # (row length, rows) of wq, wk, wv, wo
        sizes = [W.row_bytes(t, n) * r for t, (n, r) in zip(attn_types, dims)]
        per = sum((s + 255) // 256 * 256 for s in sizes)
        self.attn_bytes = sum(sizes)
        self.wbuf = torch.empty(per * n_layers + 256, dtype=torch.uint8, device=device)
        self._mats = (_lib.GGUFTensor * (4 * n_layers))()
        self._blocks = (_lib.Block * n_layers)()
        self.ones = torch.ones(head_size, dtype=torch.float32, device=device)
        s = M._stream_handle()
        off = 0
        for l in range(n_layers):
            for i, (t, (n, r)) in enumerate(zip(attn_types, dims)):
                ptr = self.wbuf.data_ptr() + off
                _lib.check(self.lib.vireo_synth_matrix_dev(t, C.c_void_p(ptr), n, 0, r, seed,
                                                           W.stream_id(l, KIND_WQ + i), 0.05, s),
                           "vireo_synth_matrix_dev")
                self._mats[4 * l + i].ggml_type = t
                self._mats[4 * l + i].data = ptr
                off += (sizes[i] + 255) // 256 * 256
            b = self._blocks[l]
            b.wq, b.wk, b.wv, b.wo = (C.pointer(self._mats[4 * l + i]) for i in range(4))
            b.q_norm = b.k_norm = self.ones.data_ptr()
            b.q_norm_len = b.k_norm_len = head_size
        self.rope = torch.empty((max_pos, head_size), dtype=torch.float32, device=device)
        _lib.check(self.lib.vireo_rope_table(C.c_float(rope_base), head_size, max_pos, C.c_void_p(self.rope.data_ptr())),
                   "vireo_rope_table")
        lm = C.pointer(self.stack._lm_t)
        self.model = _lib.Model(n_layers, d, n_heads, n_kv_heads, head_size, 0, vocab, W.EPS, rope_base,
                                self._blocks, C.pointer(self.stack.moe.model), lm, None, lm,
                                self.rope.data_ptr(), max_pos)
        self.kv = DeviceKV(n_layers * n_kv_heads, head_size, block_tokens, 32, 256, dense=True,
                           max_tokens=max_pos if contiguous else 0)
        self.pos = torch.zeros(1, dtype=torch.int32, device=device)
        nbytes = self.lib.vireo_model_state_bytes(C.byref(self.model))
        if nbytes < 0:
            raise _lib.VireoError(f"vireo_model_state_bytes failed: {nbytes}")
        self.state = torch.empty(int(nbytes), dtype=torch.uint8, device=device)
        self.x = torch.empty(d, dtype=torch.float32, device=device)
        self.logits = torch.empty(vocab, dtype=torch.float32, device=device)
        self.token = torch.full((1,), 17, dtype=torch.int32, device=device)
        self.n_layers, self.n_heads, self.n_kv_heads, self.head_size, self.vocab = (n_layers, n_heads, n_kv_heads,
                                                                                    head_size, vocab)
        torch.cuda.synchronize()

    def step(self, pos, stream=None):
        """forward(token, pos) with logits and argmax: self.token is read and overwritten."""
        _lib.check(self.lib.vireo_model_step(C.byref(self.model), C.c_void_p(self.kv.h), _ptr(self.token), pos, 1,
                                             _ptr(self.x), _ptr(self.logits), _ptr(self.state), _stream(stream)),
                   "vireo_model_step")

    def step_pos(self, stream=None):
        """vireo_model_step_pos at self.pos (device), which advances."""
        _lib.check(self.lib.vireo_model_step_pos(C.byref(self.model), C.c_void_p(self.kv.h), _ptr(self.token),
                                                 _ptr(self.pos), 1, _ptr(self.x), _ptr(self.logits), _ptr(self.state),
                                                 _stream(stream)), "vireo_model_step_pos")

    def close(self):
        if getattr(self, "kv", None):
            self.kv.close()
            self.kv = None
        if getattr(self, "stack", None):
            self.stack.close()
            self.stack = None
