"""An attention-free stack of MoE layers with a Q8_0 LM head, decoded greedily
on the GPU through moe_stack_step (the skeleton of the reference's forward,
src/gguf_run.c:216-254: residual x carried through the layers, RMSNorm before
each MoE FFN, final RMSNorm, LM head, argmax).

All norm weights are unit weights; the LM head matrix doubles as the token
embedding (a tied model, src/gguf_run.c:297), so a step starts from the
dequantized row of the previous step's token.
"""
import ctypes as C

import torch

from . import _lib
from . import moe as M
from . import workloads as W


class DeviceStack:
    def __init__(self, shape, n_layers, vocab=W.LM_VOCAB, seed=1234, lm_type=W.Q8_0, device="cuda"):
        self.lib = _lib.load()
        self.shape, self.n_layers, self.vocab, self.seed, self.lm_type = shape, n_layers, vocab, seed, lm_type
        self.moe = M.DeviceMoE(shape, n_layers, seed=seed, device=device)
        d = shape.d
        rb = W.row_bytes(lm_type, d)
        self.lm = torch.empty(rb * vocab + 256, dtype=torch.uint8, device=device)
        _lib.check(self.lib.vireo_synth_matrix_dev(lm_type, C.c_void_p(self.lm.data_ptr()), d, 0, vocab, seed,
                                                   W.stream_id(0, W.KIND_LM_HEAD), W.WEIGHT_SIGMA,
                                                   M._stream_handle()), "vireo_synth_matrix_dev")
        torch.cuda.synchronize()
        self._lm_t = _lib.GGUFTensor()
        self._lm_t.ggml_type = lm_type
        self._lm_t.data = self.lm.data_ptr()
        self.st = _lib.MoEStack(C.pointer(self.moe.model), None, None, C.pointer(self._lm_t), vocab, W.EPS)
        self.x = torch.empty(d, dtype=torch.float32, device=device)
        self.xb = torch.empty(d, dtype=torch.float32, device=device)
        self.logits = torch.empty(vocab, dtype=torch.float32, device=device)

    def step(self, token, stream=None):
        """One decode step: token (device int32 [1]) is read and overwritten
        with the next token; self.x / self.logits hold that step's residual
        and logits."""
        _lib.check(self.lib.moe_stack_step(C.byref(self.st), M._ptr(token), M._ptr(self.x), M._ptr(self.xb),
                                           M._ptr(self.logits), M._stream_handle(stream)), "moe_stack_step")

    def step_trace(self, token, idx, flags, stream=None):
        """step() that also records every layer's routing: idx (device int32
        [layers x k]) and flags (device uint32 [layers])."""
        _lib.check(self.lib.moe_stack_step_trace(C.byref(self.st), M._ptr(token), M._ptr(self.x), M._ptr(self.xb),
                                                 M._ptr(self.logits), M._ptr(idx), M._ptr(flags),
                                                 M._stream_handle(stream)), "moe_stack_step_trace")

    def device_lm_head(self):
        """The LM head's bytes copied from HBM (host uint8)."""
        return self.lm[:W.row_bytes(self.lm_type, self.shape.d) * self.vocab].cpu().numpy()

    def host_lm_head(self):
        return W.host_matrix(self.lm_type, self.shape.d, 0, self.vocab, self.seed, W.stream_id(0, W.KIND_LM_HEAD))

    def close(self):
        self.moe.close()
