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

    def __init__(self, path, max_pos=256, expert_capacity=0, block_tokens=32, device="cuda"):
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
        self.kv = DeviceKV(self.n_layers * self.n_kv_heads, self.head_size, block_tokens, 32, 256, dense=True)
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
