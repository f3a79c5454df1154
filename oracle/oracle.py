"""Python access to the CPU checkers -- TEST INFRASTRUCTURE ONLY.

Two libraries, both built by oracle/Makefile:
  liboracle.so          this build's C restatement of the reference path
                        (oracle.c, each function citing the reference lines)
  _ref/libvireo_ref.so  the reference's own sources compiled where they lie,
                        with ref_shim.c exposing its static MoE functions

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may use
this module, and only as the checker or the timed CPU baseline -- never as the
thing that produces a product result.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libvireo_ref.so")

F32, F16, Q5_0, Q8_0, Q4_K, Q6_K = 0, 1, 6, 8, 12, 14
_vp = C.c_void_p


class _GStr(C.Structure):
    _fields_ = [("ptr", C.c_char_p), ("len", C.c_uint64)]


class _GTensor(C.Structure):  # src/gguf.h:36-45
    _fields_ = [("name", _GStr), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 4), ("ggml_type", C.c_uint32),
                ("offset", C.c_uint64), ("data", _vp), ("n_elems", C.c_uint64), ("nbytes", C.c_uint64)]


class _MoeCfg(C.Structure):
    _fields_ = [("d", C.c_int), ("ne", C.c_int), ("k", C.c_int), ("fe", C.c_int), ("renorm", C.c_int),
                ("gate_type", C.c_uint32), ("up_type", C.c_uint32), ("down_type", C.c_uint32)]


def _ptr(a):
    return a.ctypes.data_as(_vp) if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(np.frombuffer(a, dtype=np.uint8) if isinstance(a, (bytes, bytearray)) else a,
                                dtype=np.uint8)


class Oracle:
    """The C restatement (liboracle.so)."""

    def __init__(self, path=ORACLE_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        L.or_f16_to_f32.restype = C.c_float
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_dequant_row.argtypes = [C.c_uint32, _vp, _vp, C.c_int]
        L.or_matmul.argtypes = [_vp, _vp, C.c_uint32, _vp, C.c_int, C.c_int]
        L.or_rmsnorm.argtypes = [_vp, _vp, _vp, C.c_int, C.c_float]
        L.or_softmax.argtypes = [_vp, C.c_int]
        L.or_topk.argtypes = [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp]
        L.or_argmax.restype = C.c_int
        L.or_argmax.argtypes = [_vp, C.c_int]
        L.or_moe_ffn.argtypes = [C.POINTER(_MoeCfg), _vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_int, _vp, _vp, _vp]
        L.or_store_create.restype = _vp
        L.or_store_create.argtypes = [C.c_int, C.c_uint64, C.c_int, C.c_int]
        L.or_store_register.argtypes = [_vp, C.c_int, C.c_int, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32,
                                        C.c_uint32, C.c_uint32]
        L.or_store_lookup.restype = C.c_int
        L.or_store_lookup.argtypes = [_vp, C.c_int, C.c_int, _vp]
        L.or_store_release.argtypes = [_vp, _vp]
        L.or_store_stats.argtypes = [_vp, _vp]
        L.or_store_destroy.argtypes = [_vp]

    def f16_to_f32(self, h):
        return np.float32(self.lib.or_f16_to_f32(int(h)))

    def dequant_row(self, typ, src, n):
        src = _u8(src)
        out = np.empty(n, np.float32)
        self.lib.or_dequant_row(typ, _ptr(src), _ptr(out), n)
        return out

    def matmul(self, typ, w, x, n, d):
        w = _u8(w) if typ != F32 else _f32(w)
        x = _f32(x)
        y = np.empty(d, np.float32)
        self.lib.or_matmul(_ptr(y), _ptr(x), typ, _ptr(w), n, d)
        return y

    def rmsnorm(self, x, w, eps):
        x, w = _f32(x), _f32(w)
        o = np.empty_like(x)
        self.lib.or_rmsnorm(_ptr(o), _ptr(x), _ptr(w), x.size, eps)
        return o

    def softmax(self, v):
        v = _f32(v).copy()
        self.lib.or_softmax(_ptr(v), v.size)
        return v

    def topk(self, p, k, renorm):
        p = _f32(p)
        kk = min(k, 64)
        idx = np.empty(kk, np.int32)
        w = np.empty(kk, np.float32)
        self.lib.or_topk(_ptr(p), p.size, k, int(renorm), _ptr(idx), _ptr(w))
        return idx, w

    def argmax(self, v):
        v = _f32(v)
        return self.lib.or_argmax(_ptr(v), v.size)

    def moe_ffn(self, shape, router, gate, up, down, x, hb, bias=None):
        """moe_ffn over T tokens. gate/up/down: lists of per-expert byte arrays
        (None = unregistered). Returns (x_out, idx, w, probs)."""
        d, E, k, fe = shape.d, shape.E, shape.k, shape.fe
        cfg = _MoeCfg(d, E, k, fe, int(shape.renorm), shape.gate_type, shape.up_type, shape.down_type)
        x = _f32(x).reshape(-1, d).copy()
        hb = _f32(hb).reshape(-1, d)
        T = x.shape[0]
        router = _f32(router)
        keep = [[_u8(a) if a is not None else None for a in lst] for lst in (gate, up, down)]
        tabs = [(_vp * E)(*[(a.ctypes.data if a is not None else None) for a in lst]) for lst in keep]
        kk = min(k, 64)
        idx = np.empty((T, kk), np.int32)
        w = np.empty((T, kk), np.float32)
        probs = np.empty((T, E), np.float32)
        b = _f32(bias) if bias is not None else None
        self.lib.or_moe_ffn(C.byref(cfg), _ptr(router), _ptr(b), C.cast(tabs[0], _vp), C.cast(tabs[1], _vp),
                            C.cast(tabs[2], _vp), _ptr(x), _ptr(hb), T, _ptr(idx), _ptr(w), _ptr(probs))
        return x, idx, w, probs

    # lease-LRU pager restatement
    def store_create(self, fd, cap, n_layers, n_experts):
        return self.lib.or_store_create(fd, cap, n_layers, n_experts)

    def store_register(self, s, l, e, go, uo, do, gb, ub, db):
        self.lib.or_store_register(s, l, e, go, uo, do, gb, ub, db)

    def store_lookup(self, s, l, e):
        view = (_vp * 4)()
        rc = self.lib.or_store_lookup(s, l, e, C.cast(view, _vp))
        return rc, view

    def store_release(self, s, view):
        self.lib.or_store_release(s, C.cast(view, _vp))

    def store_stats(self, s):
        out = (C.c_uint64 * 7)()
        self.lib.or_store_stats(s, C.cast(out, _vp))
        return list(out)

    def store_destroy(self, s):
        self.lib.or_store_destroy(s)


class Reference:
    """The reference's own code compiled from /root/reference (oracle/_ref)."""

    @staticmethod
    def available(path=REF_LIB):
        return os.path.exists(path)

    def __init__(self, path=REF_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle ref` where the reference is mounted")
        L = self.lib = C.CDLL(path)
        L.gguf_f16_to_f32.restype = C.c_float
        L.gguf_f16_to_f32.argtypes = [C.c_uint16]
        L.gguf_dequant_row.argtypes = [C.c_uint32, _vp, _vp, C.c_int]
        L.gguf_matmul.argtypes = [_vp, _vp, C.POINTER(_GTensor), C.c_int, C.c_int]
        L.ref_rmsnorm.argtypes = [_vp, _vp, _vp, C.c_int, C.c_float]
        L.ref_softmax_n.argtypes = [_vp, C.c_int]
        L.ref_argmax.restype = C.c_int
        L.ref_argmax.argtypes = [_vp, C.c_int]
        L.ref_moe_create.restype = _vp
        L.ref_moe_create.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _vp, C.c_uint32,
                                     C.c_uint32, C.c_uint32, _vp, _vp, _vp, C.c_uint64, C.c_uint64, C.c_uint64,
                                     C.c_uint64]
        L.ref_moe_run.restype = C.c_int
        L.ref_moe_run.argtypes = [_vp, C.c_int, _vp, _vp, C.c_int, _vp, _vp]
        L.ref_moe_stats.argtypes = [_vp, _vp]
        L.ref_moe_destroy.argtypes = [_vp]
        L.expert_store_create.restype = _vp
        L.expert_store_create.argtypes = [C.c_int, C.c_uint64, C.c_int, C.c_int]
        L.expert_store_register.argtypes = [_vp, C.c_int, C.c_int, _vp]
        L.expert_store_lookup.restype = C.c_int
        L.expert_store_lookup.argtypes = [_vp, C.c_int, C.c_int, _vp]
        L.expert_store_release.argtypes = [_vp, _vp]
        L.expert_store_stats.argtypes = [_vp, _vp]
        L.expert_store_destroy.argtypes = [_vp]

    def f16_to_f32(self, h):
        return np.float32(self.lib.gguf_f16_to_f32(int(h)))

    def dequant_row(self, typ, src, n):
        src = _u8(src)
        out = np.empty(n, np.float32)
        self.lib.gguf_dequant_row(typ, _ptr(src), _ptr(out), n)
        return out

    def matmul(self, typ, w, x, n, d):
        w = _u8(w) if typ != F32 else _f32(w)
        x = _f32(x)
        y = np.empty(d, np.float32)
        t = _GTensor()
        t.data = w.ctypes.data
        t.ggml_type = typ
        self.lib.gguf_matmul(_ptr(y), _ptr(x), C.byref(t), n, d)
        return y

    def rmsnorm(self, x, w, eps):
        x, w = _f32(x), _f32(w)
        o = np.empty_like(x)
        self.lib.ref_rmsnorm(_ptr(o), _ptr(x), _ptr(w), x.size, eps)
        return o

    def softmax(self, v):
        v = _f32(v).copy()
        self.lib.ref_softmax_n(_ptr(v), v.size)
        return v

    def argmax(self, v):
        v = _f32(v)
        return self.lib.ref_argmax(_ptr(v), v.size)


class RefMoE:
    """A reference MoE model: moe_ffn + ExpertStore over a temp backing file."""

    def __init__(self, ref, shape, routers, gate_all, up_all, down_all, cap_bytes=0):
        """routers: list (per layer) of [E, d] F32; *_all: list (per layer) of
        stacked expert byte arrays [E * slice]."""
        self.ref, self.shape = ref, shape
        L = len(routers)
        self._keep = [_f32(r) for r in routers], [_u8(a) for a in gate_all], [_u8(a) for a in up_all], \
            [_u8(a) for a in down_all]
        rt = (_vp * L)(*[a.ctypes.data for a in self._keep[0]])
        gt = (_vp * L)(*[a.ctypes.data for a in self._keep[1]])
        ut = (_vp * L)(*[a.ctypes.data for a in self._keep[2]])
        dt = (_vp * L)(*[a.ctypes.data for a in self._keep[3]])
        E = shape.E
        self.h = ref.lib.ref_moe_create(L, shape.d, E, shape.k, shape.fe, int(shape.renorm), C.cast(rt, _vp),
                                        shape.gate_type, shape.up_type, shape.down_type, C.cast(gt, _vp),
                                        C.cast(ut, _vp), C.cast(dt, _vp), self._keep[1][0].size // E,
                                        self._keep[2][0].size // E, self._keep[3][0].size // E, cap_bytes)
        if not self.h:
            raise RuntimeError("ref_moe_create failed")

    def run(self, layer, x, hb):
        d, E, k = self.shape.d, self.shape.E, min(self.shape.k, 64)
        x = _f32(x).reshape(-1, d).copy()
        hb = _f32(hb).reshape(-1, d)
        T = x.shape[0]
        idx = np.empty((T, k), np.int32)
        probs = np.empty((T, E), np.float32)
        rc = self.ref.lib.ref_moe_run(self.h, layer, _ptr(x), _ptr(hb), T, _ptr(idx), _ptr(probs))
        if rc:
            raise RuntimeError(f"ref_moe_run failed: {rc}")
        return x, idx, probs

    def stats(self):
        out = (C.c_uint64 * 7)()
        self.ref.lib.ref_moe_stats(self.h, C.cast(out, _vp))
        return list(out)

    def close(self):
        if self.h:
            self.ref.lib.ref_moe_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _KVConfig(C.Structure):  # src/kvstore.h:26-33
    _fields_ = [("n_layers", C.c_int), ("kv_dim", C.c_int), ("block_tokens", C.c_int), ("sink_tokens", C.c_int),
                ("window_tokens", C.c_int), ("capacity_bytes", C.c_uint64)]


class _KVStats(C.Structure):  # src/kvstore.h:35-44
    _fields_ = [(n, C.c_uint64) for n in ("requests", "hits", "misses", "prefetched", "bytes_read", "bytes_spilled",
                                          "resident_bytes", "capacity_bytes")]


_KV_APPEND = C.CFUNCTYPE(None, _vp, C.c_int, C.c_int, _vp, _vp)
_KV_ATTEND = C.CFUNCTYPE(None, _vp, C.c_int, _vp, _vp)
_KV_STATS = C.CFUNCTYPE(None, _vp, _vp)
_KV_DESTROY = C.CFUNCTYPE(None, _vp)


class _KVOps(C.Structure):  # src/kvstore.h:47-52
    _fields_ = [("append", _KV_APPEND), ("attend", _KV_ATTEND), ("stats", _KV_STATS), ("destroy", _KV_DESTROY)]


class _KVStore(C.Structure):  # src/kvstore.h:54-58
    _fields_ = [("ops", C.POINTER(_KVOps)), ("cfg", _KVConfig), ("state", _vp)]


class _SelectStrategy(C.Structure):  # src/select/select.h:38-44
    _fields_ = [("name", C.c_char_p), ("select", _vp), ("budget", C.c_int)]


class RefKV:
    """The reference's own KV stores (src/kvstore_dense.c, src/kvstore_ooc.c
    with src/select/*), compiled into oracle/_ref: strategy "all", "recent"
    or "topk" (with budget) for the out-of-core store, None for the dense one.
    append/attend take numpy float32 vectors."""

    def __init__(self, ref, n_layers, kv_dim, block_tokens, sink_tokens=0, window_tokens=0, capacity_bytes=0,
                 strategy=None, budget=0, workdir=None):
        L = self.lib = ref.lib
        L.kvstore_dense_create.restype = C.POINTER(_KVStore)
        L.kvstore_dense_create.argtypes = [_KVConfig]
        L.kvstore_ooc_create.restype = C.POINTER(_KVStore)
        L.kvstore_ooc_create.argtypes = [_KVConfig, _vp, C.c_char_p]
        L.vireo_select_topk.restype = _vp
        L.vireo_select_topk.argtypes = [C.c_int]
        cfg = _KVConfig(n_layers, kv_dim, block_tokens, sink_tokens, window_tokens, capacity_bytes)
        if strategy is None:
            self.s = L.kvstore_dense_create(cfg)
        else:
            if strategy == "topk":
                st = L.vireo_select_topk(budget)
            else:
                st = C.addressof(_SelectStrategy.in_dll(L, {"all": "VIREO_SELECT_ALL",
                                                            "recent": "VIREO_SELECT_RECENT"}[strategy]))
            self.s = L.kvstore_ooc_create(cfg, st, (workdir or os.environ.get("TMPDIR", "/tmp")).encode())
        self.ops = self.s.contents.ops.contents
        self.kv_dim = kv_dim

    def append(self, layer, pos, k, v):
        k, v = _f32(k), _f32(v)
        self.ops.append(C.cast(self.s, _vp), layer, pos, _ptr(k), _ptr(v))

    def attend(self, layer, q):
        q = _f32(q)
        out = np.empty(self.kv_dim, np.float32)
        self.ops.attend(C.cast(self.s, _vp), layer, _ptr(q), _ptr(out))
        return out

    def stats(self):
        st = _KVStats()
        self.ops.stats(C.cast(self.s, _vp), C.cast(C.pointer(st), _vp))
        return {n: getattr(st, n) for n, _ in _KVStats._fields_}

    def close(self):
        if getattr(self, "s", None):
            self.ops.destroy(C.cast(self.s, _vp))
            self.s = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class RefModel:
    """The reference's forward() (src/gguf_run.c:216-251) on a GGUF file
    (oracle/_ref: the shim binds the reference's Model with its own reader,
    ExpertStore and out-of-core KV store with the "all" strategy)."""

    def __init__(self, ref, path, block_tokens=32):
        L = self.lib = ref.lib
        L.ref_model_open.restype = _vp
        L.ref_model_open.argtypes = [C.c_char_p, C.c_int]
        L.ref_model_shape.argtypes = [_vp, _vp]
        L.ref_model_forward.argtypes = [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp]
        L.ref_model_close.argtypes = [_vp]
        self.h = L.ref_model_open(str(path).encode(), block_tokens)
        if not self.h:
            raise RuntimeError(f"the reference cannot bind {path}")
        sh = np.zeros(7, np.int32)
        L.ref_model_shape(self.h, _ptr(sh))
        self.dim, self.vocab, self.n_layers, self.n_heads, self.n_kv_heads, self.head_size, self.is_moe = map(int, sh)

    def forward(self, token, pos, want_logits=True):
        """(x after the last block, logits or None)."""
        x = np.empty(self.dim, np.float32)
        lg = np.empty(self.vocab, np.float32) if want_logits else None
        self.lib.ref_model_forward(self.h, int(token), int(pos), int(want_logits), _ptr(x),
                                   _ptr(lg) if want_logits else None)
        return x, lg

    def close(self):
        if getattr(self, "h", None):
            self.lib.ref_model_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
