"""The C-ABI library without a GPU: it loads, exports every function that
include/*.h declares, and its argument checks reject bad calls before any
device work. No compute entry point is called here."""
import ctypes as C
import errno
import os
import re

import numpy as np
import pytest

from vireo_amd import _lib
from vireo_amd import workloads as W

INCLUDE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")


def declared_functions():
    names = set()
    for fn in sorted(os.listdir(INCLUDE)):
        if not fn.endswith(".h"):
            continue
        src = open(os.path.join(INCLUDE, fn)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        src = re.sub(r"#[^\n]*", "", src)
        src = re.sub(r"typedef[^;]*?\{[^{}]*\}[^;]*;", "", src, flags=re.S)
        src = re.sub(r"typedef[^;]*;", "", src)
        for m in re.finditer(r"([A-Za-z_]\w*)\s*\(([^;{}]*)\)\s*;", src):
            names.add(m.group(1))
    return names


def test_header_parse_finds_the_entry_points():
    names = declared_functions()
    for n in ("moe_ffn_forward", "qmatvec", "moe_route", "moe_dispatch", "expert_store_lookup",
              "expert_store_create_device", "vireo_synth_matrix", "vireo_rmsnorm"):
        assert n in names
    assert len(names) >= 25


# The reference's GGUF reader (src/gguf.h:57-72): include/vireo_gguf.h declares
# it too, so that either header may be included first, but src/gguf.c defines
# it; the library exports its own reader as vireo_gguf_* and must not clash.
REFERENCE_READER = {"gguf_open", "gguf_close", "gguf_find", "gguf_get_u64", "gguf_get_f32", "gguf_get_str",
                    "gguf_tensor_by_name", "gguf_type_block", "gguf_dump"}


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert REFERENCE_READER <= names
    missing = [n for n in sorted(names - REFERENCE_READER) if not hasattr(lib, n)]
    assert not missing, f"declared in include/*.h but not exported: {missing}"
    clashing = [n for n in sorted(REFERENCE_READER) if hasattr(lib, n)]
    assert not clashing, f"the reference's reader must stay the reference's: {clashing}"


def test_bindings_cover_the_headers():
    assert declared_functions() - REFERENCE_READER <= set(_lib.SIGNATURES)


def test_type_block_table(lib):
    be, bb = C.c_int(), C.c_int()
    for t, (e, b) in W.BLOCK.items():
        assert lib.vireo_type_block(t, C.byref(be), C.byref(bb)) == 0
        assert (be.value, bb.value) == (e, b)
    assert lib.vireo_type_block(13, C.byref(be), C.byref(bb)) == -errno.EINVAL  # Q5_K: not on this path
    for t, (e, b) in W.BLOCK.items():
        assert lib.vireo_row_bytes(t, 512) == 512 // e * b
    assert lib.vireo_row_bytes(W.Q4_K, 100) == -errno.EINVAL


def test_strerror(lib):
    assert lib.vireo_hip_strerror(0) == b"ok"
    for e in (errno.EINVAL, errno.ENOMEM, errno.ENOSPC, errno.E2BIG):
        assert lib.vireo_hip_strerror(-e)


def test_argument_checks_before_device_work(lib):
    EINVAL = -errno.EINVAL
    assert lib.vireo_hip_set_path(6) == EINVAL and lib.vireo_hip_set_path(-1) == EINVAL
    assert lib.vireo_hip_set_path(0) == 0
    assert lib.moe_ffn_forward(None, 0, None, None, 1, None, None, None) == EINVAL
    assert lib.moe_route(None, 0, None, 1, None, None, None, None, None) == EINVAL
    assert lib.moe_dispatch(None, 1, 0, 8, None, None, None, None) == EINVAL
    assert lib.moe_dispatch(None, 1, 2, 300, None, None, None, None) == EINVAL
    t = _lib.GGUFTensor()
    t.ggml_type = W.Q4_K
    t.data = 0x1008  # not 16-byte aligned
    y = C.c_void_p(0x2000)
    assert lib.qmatvec_async(y, y, C.byref(t), 256, 4, None) == EINVAL
    t.data = 0x1000
    assert lib.qmatvec_async(y, y, C.byref(t), 100, 4, None) == EINVAL  # n not a multiple of 256
    t.ggml_type = 13
    assert lib.qmatvec_async(y, y, C.byref(t), 256, 4, None) == EINVAL
    assert lib.qdequant_rows(W.Q8_0, None, None, 32, -1, None) == EINVAL


def test_model_checks(lib):
    """A model whose layer is malformed is refused before anything runs."""
    tr = _lib.GGUFTensor()
    tr.ggml_type = W.Q8_0  # router must be F32
    tr.data = 0x1000
    layers = (_lib.MoELayer * 1)()
    layers[0].router = C.pointer(tr)
    m = _lib.MoEModel(2048, 64, 8, 1024, 0, 1, layers, None)
    x = C.c_void_p(0x4000)
    assert lib.moe_ffn_forward(C.byref(m), 0, x, x, 1, None, None, None) == -errno.EINVAL
    tr.ggml_type = W.F32
    assert lib.moe_ffn_forward(C.byref(m), 1, x, x, 1, None, None, None) == -errno.EINVAL  # layer out of range
    m.n_used = 0
    assert lib.moe_ffn_forward(C.byref(m), 0, x, x, 1, None, None, None) == -errno.EINVAL
    m.n_used, m.n_experts = 8, 257
    assert lib.moe_ffn_forward(C.byref(m), 0, x, x, 1, None, None, None) == -errno.EINVAL
    m.n_experts = 64
    # no expert tensors / store
    assert lib.moe_ffn_forward(C.byref(m), 0, x, x, 1, None, None, None) == -errno.EINVAL
    assert lib.moe_ffn_forward(C.byref(m), 0, x, x, 0, None, None, None) == 0  # no tokens: nothing to do


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.VireoError):
        _lib.load()


def test_quantize_rejects_bad_shapes(lib):
    src = np.zeros(100, np.float32)
    dst = np.zeros(1000, np.uint8)
    assert lib.vireo_quantize(W.Q4_K, src.ctypes.data_as(C.c_void_p), dst.ctypes.data_as(C.c_void_p), 100, 1) \
        == -errno.EINVAL
