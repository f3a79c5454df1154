"""Host-side mirror of the reference's MoE interface over the vireo-hip C-ABI.

DeviceMoE holds what moe_ffn reads from the reference's Model and Layer
(src/gguf_run.c:141-157): the MoE hyper-parameters, per-layer router and
expert tensors, and an ExpertStore whose resident pool is HBM. forward()
is moe_ffn (src/gguf_run.c:185-214) for a batch of independent tokens:
x[t] += moe(hb[t]) in place. PyTorch only provides device memory and the
stream; all compute is in libvireo_hip.so.
"""
import ctypes as C

import numpy as np
import torch

from . import _lib
from . import workloads as W

# words of stamps per call of moe_decode_phases: [3 kernels][256 workgroups][8 phases]
PHASE_WORDS = 3 * 256 * 8


def _stream_handle(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream) if s.cuda_stream else None


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _need(name, t, rows, cols, dtype=torch.float32):
    """The library takes raw device pointers: check sizes on the host."""
    if t is None or t.dtype != dtype or not t.is_cuda or not t.is_contiguous() or t.numel() < rows * cols or \
            (t.dim() >= 1 and t.shape[-1] != cols and t.dim() > 1):
        raise ValueError(f"{name}: need a contiguous {dtype} device tensor of at least [{rows} x {cols}], "
                         f"got {None if t is None else (tuple(t.shape), t.dtype, t.device)}")


class DeviceMoE:
    """n_layers MoE layers of `shape`, all experts resident in HBM.

    Expert bytes are generated on the GPU straight into one device buffer laid
    out per layer as [gate_exps | up_exps | down_exps] (GGUF's stacked expert
    tensors); an ExpertStore over that buffer makes every slice resident
    without a copy, and moe_ffn_forward pins each layer's leases on first use.
    """

    def __init__(self, shape, n_layers=1, seed=1234, logit_bias=None, device="cuda", layer_seeds=None,
                 unregistered=()):
        self.lib = _lib.load()
        self.shape, self.n_layers, self.seed = shape, n_layers, seed
        self.layer_seeds = layer_seeds or [(seed, l) for l in range(n_layers)]
        E, d, fe = shape.E, shape.d, shape.fe
        gs, us, ds = shape.slice_bytes()
        self.slices = (gs, us, ds)
        self.layer_bytes = E * (gs + us + ds)
        total = self.layer_bytes * n_layers
        self.buf = torch.empty(total + 256, dtype=torch.uint8, device=device)
        base = self.buf.data_ptr()
        s = _stream_handle()
        for l, (lseed, lid) in enumerate(self.layer_seeds):
            off = l * self.layer_bytes
            for kind, typ, n, rows, at in ((W.KIND_GATE, shape.gate_type, d, E * fe, off),
                                           (W.KIND_UP, shape.up_type, d, E * fe, off + E * gs),
                                           (W.KIND_DOWN, shape.down_type, fe, E * d, off + E * (gs + us))):
                _lib.check(self.lib.vireo_synth_matrix_dev(typ, C.c_void_p(base + at), n, 0, rows, lseed,
                                                           W.stream_id(lid, kind), W.WEIGHT_SIGMA, s),
                           "vireo_synth_matrix_dev")
        self.routers = torch.empty((n_layers, E, d), dtype=torch.float32, device=device)
        for l, (lseed, lid) in enumerate(self.layer_seeds):
            r = W.host_normal(E * d, lseed, W.stream_id(lid, W.KIND_ROUTER), sigma=W.WEIGHT_SIGMA)
            self.routers[l].copy_(torch.from_numpy(r.reshape(E, d)))
        self.bias = None
        if logit_bias is not None:
            self.bias = torch.as_tensor(np.asarray(logit_bias, np.float32)).to(device)
        torch.cuda.synchronize()
        self.es = self.lib.expert_store_create_device(C.c_void_p(base), total, 0, n_layers, E)
        if not self.es:
            raise _lib.VireoError("expert_store_create_device failed")
        for l in range(n_layers):
            off = l * self.layer_bytes
            for e in range(E):
                if (l, e) in unregistered:  # its lookups fail, as for an expert missing from the file
                    continue
                sl = _lib.ExpertSlices(off + e * gs, off + E * gs + e * us, off + E * (gs + us) + e * ds, gs, us, ds)
                self.lib.expert_store_register(self.es, l, e, C.byref(sl))
        # tensors and the model struct the C-ABI reads
        self._tensors = []
        layers = (_lib.MoELayer * n_layers)()
        for l in range(n_layers):
            tr = _lib.GGUFTensor()
            tr.ggml_type = W.F32
            tr.data = self.routers[l].data_ptr()
            tg, tu, td = _lib.GGUFTensor(), _lib.GGUFTensor(), _lib.GGUFTensor()
            tg.ggml_type, tu.ggml_type, td.ggml_type = shape.gate_type, shape.up_type, shape.down_type
            self._tensors += [tr, tg, tu, td]
            layers[l].router = C.pointer(tr)
            layers[l].gate_exps = C.pointer(tg)
            layers[l].up_exps = C.pointer(tu)
            layers[l].down_exps = C.pointer(td)
            layers[l].logit_bias = self.bias.data_ptr() if self.bias is not None else None
        self._layers = layers
        self.model = _lib.MoEModel(d, E, shape.k, fe, int(shape.renorm), n_layers, layers, self.es)

    # -- the three stages and the whole layer --------------------------------
    def route(self, layer, hb, stream=None, want_probs=False):
        T = hb.shape[0]
        k = self.shape.k
        _need("hb", hb, T, self.shape.d)
        idx = torch.empty((T, k), dtype=torch.int32, device=hb.device)
        w = torch.empty((T, k), dtype=torch.float32, device=hb.device)
        flags = torch.empty(T, dtype=torch.int32, device=hb.device)
        probs = torch.empty((T, self.shape.E), dtype=torch.float32, device=hb.device) if want_probs else None
        _lib.check(self.lib.moe_route(C.byref(self.model), layer, _ptr(hb), T, _ptr(idx), _ptr(w), _ptr(flags),
                                      _ptr(probs), _stream_handle(stream)), "moe_route")
        return idx, w, flags, probs

    def forward(self, layer, x, hb, stream=None, return_routing=False):
        """x[t] += moe(hb[t]) in place for every token t (moe_ffn_forward)."""
        T = hb.shape[0]
        _need("hb", hb, T, self.shape.d)
        _need("x", x, T, self.shape.d)
        idx = w = None
        if return_routing:
            idx = torch.empty((T, self.shape.k), dtype=torch.int32, device=hb.device)
            w = torch.empty((T, self.shape.k), dtype=torch.float32, device=hb.device)
        _lib.check(self.lib.moe_ffn_forward(C.byref(self.model), layer, _ptr(x), _ptr(hb), T, _ptr(idx), _ptr(w),
                                            _stream_handle(stream)), "moe_ffn_forward")
        return (idx, w) if return_routing else None

    def decode_state(self):
        """A device buffer for moe_decode_stage (one layer, one token)."""
        nb = self.lib.moe_decode_state_bytes(C.byref(self.model))
        if nb < 0:
            raise _lib.VireoError(f"no decode plan for {self.shape.name}")
        return torch.empty(int(nb), dtype=torch.uint8, device=self.buf.device)

    def decode_stage(self, layer, stage, x, hb, state, idx=None, w=None, stream=None):
        """One stage (0 route, 1 top-k + gate/up, 2 down + combine) of the
        one-token decode plan over `state`."""
        d, k = self.shape.d, self.shape.k
        _need("hb", hb, 1, d)
        if stage == 2:
            _need("x", x, 1, d)
        for name, t, dt in (("idx", idx, torch.int32), ("w", w, torch.float32)):
            if t is not None:
                _need(name, t, 1, k, dt)
        nb = self.lib.moe_decode_state_bytes(C.byref(self.model))
        if state.numel() < nb or state.dtype != torch.uint8:
            raise ValueError(f"state: need {nb} bytes")
        _lib.check(self.lib.moe_decode_stage(C.byref(self.model), layer, stage, _ptr(x), _ptr(hb), _ptr(state),
                                             _ptr(idx), _ptr(w), _stream_handle(stream)), "moe_decode_stage")

    def decode_stage_timed(self, stage, layers, x, hb, states, idx, w, stream=None):
        """Launch `stage` once per entry of `layers` (token row i of x/hb,
        state i of the [n x stride] uint8 tensor `states`) back to back and
        return each launch's kernel duration in microseconds."""
        n = len(layers)
        d, k = self.shape.d, self.shape.k
        # the library sees raw pointers: every buffer must hold n rows
        for name, t, cols in (("x", x, d), ("hb", hb, d), ("idx", idx, k), ("w", w, k)):
            if t is None or t.dim() != 2 or t.shape[0] < n or t.shape[1] != cols or not t.is_contiguous():
                raise ValueError(f"decode_stage_timed: {name} must be a contiguous [>= {n} x {cols}] tensor")
        if states.dim() != 2 or states.shape[0] < n:
            raise ValueError(f"decode_stage_timed: states must hold {n} states")
        if any(not 0 <= l < self.n_layers for l in layers):
            raise ValueError("decode_stage_timed: layer out of range")
        lay = (C.c_int * n)(*layers)
        us = (C.c_float * n)()
        _lib.check(self.lib.moe_decode_stage_timed(C.byref(self.model), stage, n, lay, _ptr(x), _ptr(hb),
                                                   _ptr(states), states.stride(0), _ptr(idx), _ptr(w), us,
                                                   _stream_handle(stream)), "moe_decode_stage_timed")
        return np.array(us[:], dtype=np.float64)

    def decode_phases(self, layers, x, hb, stream=None, stamps=None):
        """Enqueue one moe_ffn_forward call per entry of `layers` (token row i
        of x / hb) with the decode kernels recording per-workgroup phase stamps
        (moe_decode_phases) into `stamps`, a zeroed int64 tensor of
        [n x PHASE_WORDS] (made here when None); returns it. The caller reads
        it after synchronising (or after replaying a graph that captured it)."""
        n = len(layers)
        d = self.shape.d
        for name, t in (("x", x), ("hb", hb)):
            if t is None or t.dim() != 2 or t.shape[0] < n or t.shape[1] != d or not t.is_contiguous():
                raise ValueError(f"decode_phases: {name} must be a contiguous [>= {n} x {d}] tensor")
        if any(not 0 <= l < self.n_layers for l in layers):
            raise ValueError("decode_phases: layer out of range")
        if stamps is None:
            stamps = torch.zeros((n, PHASE_WORDS), dtype=torch.int64, device=x.device)
        if stamps.dim() != 2 or stamps.shape[0] < n or stamps.shape[1] != PHASE_WORDS or not stamps.is_contiguous():
            raise ValueError(f"decode_phases: stamps must be a contiguous [>= {n} x {PHASE_WORDS}] int64 tensor")
        lay = (C.c_int * n)(*layers)
        _lib.check(self.lib.moe_decode_phases(C.byref(self.model), n, lay, _ptr(x), _ptr(hb), _ptr(stamps),
                                              _stream_handle(stream)), "moe_decode_phases")
        return stamps

    def decode_states(self, n):
        """n decode states, one per row of a [n x stride] uint8 tensor."""
        nb = self.lib.moe_decode_state_bytes(C.byref(self.model))
        if nb < 0:
            raise _lib.VireoError(f"no decode plan for {self.shape.name}")
        stride = (int(nb) + 255) // 256 * 256
        buf = torch.empty(n * stride + 256, dtype=torch.uint8, device=self.buf.device)
        off = (-buf.data_ptr()) % 256
        return buf[off:off + n * stride].view(n, stride)

    def stats(self):
        """The reference's ExpertStats for the work done so far (expert_store_stats)."""
        st = _lib.ExpertStats()
        self.lib.expert_store_stats(self.es, C.byref(st))
        return {n: getattr(st, n) for n, _ in _lib.ExpertStats._fields_}

    def hbm_stats(self):
        """What the HBM pool did (expert_store_hbm_stats)."""
        st = _lib.ExpertStats()
        self.lib.expert_store_hbm_stats(self.es, C.byref(st))
        return {n: getattr(st, n) for n, _ in _lib.ExpertStats._fields_}

    # -- host copies of the same bytes, for the checkers ----------------------
    def host_layer(self, layer):
        lseed, lid = self.layer_seeds[layer]
        return W.host_layer(self.shape, lid, lseed)

    def host_router(self, layer):
        return self.routers[layer].cpu().numpy()

    def expert_bytes(self, layer, e):
        """One expert's gate, up and down slices copied from HBM (host uint8)."""
        E = self.shape.E
        gs, us, ds = self.slices
        off = layer * self.layer_bytes
        g = self.buf[off + e * gs:off + (e + 1) * gs]
        u = self.buf[off + E * gs + e * us:off + E * gs + (e + 1) * us]
        d = self.buf[off + E * (gs + us) + e * ds:off + E * (gs + us) + (e + 1) * ds]
        return g.cpu().numpy(), u.cpu().numpy(), d.cpu().numpy()

    def device_layer_bytes(self, layer):
        """The layer's stacked expert bytes as stored in HBM (gate, up, down)."""
        E = self.shape.E
        gs, us, ds = self.slices
        off = layer * self.layer_bytes
        b = self.buf[off:off + self.layer_bytes].cpu().numpy()
        return b[:E * gs], b[E * gs:E * (gs + us)], b[E * (gs + us):]

    def close(self):
        if getattr(self, "es", None):
            torch.cuda.synchronize()
            self.lib.expert_store_destroy(self.es)
            self.es = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def dispatch(idx, n_experts, stream=None):
    """Bucket (token, slot) pairs by expert: (counts, offs, perm)."""
    lib = _lib.load()
    T, k = idx.shape
    counts = torch.empty(n_experts, dtype=torch.int32, device=idx.device)
    offs = torch.empty(n_experts + 1, dtype=torch.int32, device=idx.device)
    perm = torch.empty(T * k, dtype=torch.int32, device=idx.device)
    _lib.check(lib.moe_dispatch(_ptr(idx), T, k, n_experts, _ptr(counts), _ptr(offs), _ptr(perm),
                                _stream_handle(stream)), "moe_dispatch")
    return counts, offs, perm


def qmatvec(y, x, w_bytes, ggml_type, n, d, stream=None):
    """gguf_matmul on the GPU: y[:d] = W x, W = d rows of n elements."""
    lib = _lib.load()
    t = _lib.GGUFTensor()
    t.ggml_type = ggml_type
    t.data = w_bytes.data_ptr()
    _lib.check(lib.qmatvec_async(_ptr(y), _ptr(x), C.byref(t), n, d, _stream_handle(stream)), "qmatvec")


def dequant_rows(ggml_type, src, n, rows, stream=None):
    lib = _lib.load()
    out = torch.empty((rows, n), dtype=torch.float32, device=src.device)
    _lib.check(lib.qdequant_rows(ggml_type, _ptr(src), _ptr(out), n, rows, _stream_handle(stream)), "qdequant_rows")
    return out


def rmsnorm(x, w, eps=W.EPS, stream=None):
    lib = _lib.load()
    rows, n = x.shape
    out = torch.empty_like(x)
    _lib.check(lib.vireo_rmsnorm(_ptr(out), _ptr(x), _ptr(w), n, rows, eps, _stream_handle(stream)), "vireo_rmsnorm")
    return out


def argmax(v, stream=None):
    lib = _lib.load()
    out = torch.empty(1, dtype=torch.int32, device=v.device)
    _lib.check(lib.vireo_argmax(_ptr(v), v.numel(), _ptr(out), _stream_handle(stream)), "vireo_argmax")
    return out
