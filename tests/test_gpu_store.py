"""The ExpertStore with an HBM resident pool: the reference unit test's
scenario (tests/test_expert_store.c) with device-resident views, and the MoE
layer served from a file-backed store."""
import ctypes as C
import errno
import os
import tempfile

import numpy as np
import pytest
import torch

from conftest import d2h, golden
from vireo_amd import _lib
from vireo_amd import moe as M
from vireo_amd import workloads as W

pytestmark = pytest.mark.gpu


def _pattern(l, e, s, n):
    return ((l * 131 + e * 17 + s * 7 + np.arange(n)) & 0xFF).astype(np.uint8)


@pytest.fixture
def backing():
    g = golden("store.npz")
    NL, NE, capn = (int(v) for v in g["dims"])
    SZ = [int(v) for v in g["sizes"]]
    fd, path = tempfile.mkstemp()
    os.unlink(path)
    locs, off = [], 0
    for l in range(NL):
        for e in range(NE):
            loc = []
            for s, n in enumerate(SZ):
                os.pwrite(fd, _pattern(l, e, s, n).tobytes(), off)
                loc.append(off)
                off += n
            locs.append(_lib.ExpertSlices(*loc, *SZ))
    yield g, fd, NL, NE, capn, SZ, locs
    os.close(fd)


def test_store_scenario_on_device(cuda, lib, backing):
    g, fd, NL, NE, capn, SZ, locs = backing
    s = lib.expert_store_create(fd, sum(SZ) * capn, NL, NE)
    assert s
    for l in range(NL):
        for e in range(NE):
            lib.expert_store_register(s, l, e, C.byref(locs[l * NE + e]))
    v = _lib.ExpertView()
    for l in range(NL):
        for e in range(NE):
            assert lib.expert_store_lookup(s, l, e, C.byref(v)) == 0
            for si, (ptr, n) in enumerate(zip((v.gate, v.up, v.down), SZ)):
                assert ptr % 256 == 0
                np.testing.assert_array_equal(d2h(ptr, n), _pattern(l, e, si, n))
            lib.expert_store_release(s, C.byref(v))
            assert not v.gate and not v.slot
    st = _lib.ExpertStats()
    lib.expert_store_stats(s, C.byref(st))
    assert [getattr(st, f) for f, _ in _lib.ExpertStats._fields_] == [int(x) for x in g["after_sweep"]]
    pinned = _lib.ExpertView()
    assert lib.expert_store_lookup(s, 0, 0, C.byref(pinned)) == 0
    for l in range(NL):
        for e in range(1, NE):
            if lib.expert_store_lookup(s, l, e, C.byref(v)) == 0:
                lib.expert_store_release(s, C.byref(v))
    np.testing.assert_array_equal(d2h(pinned.gate, SZ[0]), _pattern(0, 0, 0, SZ[0]))
    lib.expert_store_release(s, C.byref(pinned))
    lib.expert_store_stats(s, C.byref(st))
    assert [getattr(st, f) for f, _ in _lib.ExpertStats._fields_] == [int(x) for x in g["after_flood"]]
    # an unregistered expert: -1 and a zeroed view (src/expert_store.c:75)
    s2 = lib.expert_store_create(fd, 0, 1, 4)
    v.gate = 1234
    assert lib.expert_store_lookup(s2, 0, 2, C.byref(v)) == -1
    assert not v.gate and not v.up and not v.down
    lib.expert_store_destroy(s2)
    lib.expert_store_destroy(s)


def test_pin_layer_capacity(cuda, lib, backing):
    g, fd, NL, NE, capn, SZ, locs = backing
    s = lib.expert_store_create(fd, sum(SZ) * (NE - 1), NL, NE)  # one expert short of a layer
    for l in range(NL):
        for e in range(NE):
            lib.expert_store_register(s, l, e, C.byref(locs[l * NE + e]))
    tab = C.c_void_p()
    assert lib.expert_store_pin_layer(s, 0, C.byref(tab)) == -errno.ENOSPC
    lib.expert_store_destroy(s)
    s = lib.expert_store_create(fd, sum(SZ) * NE, NL, NE)
    for l in range(NL):
        for e in range(NE):
            lib.expert_store_register(s, l, e, C.byref(locs[l * NE + e]))
    assert lib.expert_store_pin_layer(s, 1, C.byref(tab)) == 0
    ptrs = np.frombuffer(d2h(tab.value, NE * 3 * 8).tobytes(), np.uint64)
    for e in range(NE):
        np.testing.assert_array_equal(d2h(int(ptrs[3 * e + 2]), SZ[2]), _pattern(1, e, 2, SZ[2]))
    # pinning another layer evicts nothing pinned: no room left for it
    assert lib.expert_store_pin_layer(s, 2, C.byref(tab)) == -errno.ENOSPC
    assert lib.expert_store_unpin_layer(s, 1) == 0
    assert lib.expert_store_pin_layer(s, 2, C.byref(tab)) == 0
    lib.expert_store_destroy(s)


def test_moe_from_file_backed_store(cuda, lib):
    """The same layer served from HBM-resident experts paged in from a file
    gives the same bits as the device-generated store."""
    shape = W.SHAPES["olmoe-q4_k_m"]
    m = M.DeviceMoE(shape, 1, seed=61)
    x, hb = W.host_hidden(shape.d, 4, 61)
    hbt = torch.from_numpy(hb).to(cuda)
    xa = torch.from_numpy(x).to(cuda)
    m.forward(0, xa, hbt)
    gb, ub, db = m.device_layer_bytes(0)
    gs, us, ds = m.slices
    fd, path = tempfile.mkstemp()
    os.unlink(path)
    try:
        os.pwrite(fd, b"\0" * 4096 + gb.tobytes() + ub.tobytes() + db.tobytes(), 0)  # a header before the tensors
        s = lib.expert_store_create(fd, 0, 1, shape.E)
        for e in range(shape.E):
            sl = _lib.ExpertSlices(4096 + e * gs, 4096 + gb.size + e * us, 4096 + gb.size + ub.size + e * ds, gs, us, ds)
            lib.expert_store_register(s, 0, e, C.byref(sl))
        m.model.es = s
        xb = torch.from_numpy(x).to(cuda)
        m.forward(0, xb, hbt)
        np.testing.assert_array_equal(xb.cpu().numpy(), xa.cpu().numpy())
        st = _lib.ExpertStats()
        lib.expert_store_hbm_stats(s, C.byref(st))  # the pool: the whole layer, read once
        assert st.misses == shape.E and st.bytes_read == shape.E * (gs + us + ds)
        lib.expert_store_stats(s, C.byref(st))  # the reference: one lookup per (token, routed expert)
        assert st.requests == 4 * shape.k and st.misses == st.experts_resident
        assert st.hits + st.misses == st.requests
        torch.cuda.synchronize()
        lib.expert_store_destroy(s)
    finally:
        os.close(fd)
    m.model.es = m.es
    m.close()


def test_packed_copy_counts_against_capacity(cuda, lib):
    """The decode batch's tiled copy of a pinned layer is made only while the
    resident experts and the copy fit the store's capacity: one byte short
    and the calls read the GGUF rows (no copy), exactly enough and the copy
    is made and reported in resident_bytes and expert_store_packed_bytes; an
    unbounded store always makes it. The outputs are the same bits in every
    case."""
    shape = W.SHAPES["olmoe-q4_k_m"]
    T = 8
    m = M.DeviceMoE(shape, 1, seed=71)
    x, hb = W.host_hidden(shape.d, T, 71)
    hbt = torch.from_numpy(hb).to(cuda)
    ref = torch.from_numpy(x).to(cuda)
    try:
        _lib.check(lib.vireo_hip_set_packed(0), "vireo_hip_set_packed")
        m.forward(0, ref, hbt)
    finally:
        lib.vireo_hip_set_packed(1)
    gb, ub, db = m.device_layer_bytes(0)
    gs, us, ds = m.slices
    layer = shape.E * (gs + us + ds)
    # 16-row x 256-column Q4_K tiles of 2368 bytes for gate and up; Q6_K down rows
    q6 = shape.fe // 256 * 210
    pack = shape.E * (2 * (shape.fe // 16) * (shape.d // 256) * 2368 + shape.d * q6)
    fd, path = tempfile.mkstemp()
    os.unlink(path)
    try:
        os.pwrite(fd, gb.tobytes() + ub.tobytes() + db.tobytes(), 0)
        for cap, made in ((layer + pack - 1, False), (layer + pack, True), (0, True)):
            s = lib.expert_store_create(fd, cap, 1, shape.E)
            for e in range(shape.E):
                sl = _lib.ExpertSlices(e * gs, gb.size + e * us, gb.size + ub.size + e * ds, gs, us, ds)
                lib.expert_store_register(s, 0, e, C.byref(sl))
            m.model.es = s
            for rep in range(2):
                xt = torch.from_numpy(x).to(cuda)
                m.forward(0, xt, hbt)
                np.testing.assert_array_equal(xt.cpu().numpy().view(np.uint32), ref.cpu().numpy().view(np.uint32),
                                              err_msg=f"capacity {cap} call {rep}")
            packed = lib.expert_store_packed_bytes(s)
            assert packed == (pack if made else 0), (cap, packed)
            st = _lib.ExpertStats()
            lib.expert_store_hbm_stats(s, C.byref(st))
            assert st.resident_bytes == layer + packed
            assert cap == 0 or st.resident_bytes <= cap
            assert lib.expert_store_unpin_layer(s, 0) == 0
            assert lib.expert_store_packed_bytes(s) == 0
            torch.cuda.synchronize()
            lib.expert_store_destroy(s)
    finally:
        os.close(fd)
        m.model.es = m.es
        m.close()


@pytest.mark.parametrize("case", ["tiny_q4km", "tiny_q8", "olmoe_q8_0", "qwen3_q4_k_m"])
def test_golden_store_stats(cuda, lib, case):
    """The reference's own ExpertStore statistics after its moe_ffn over the
    golden tokens (an unbounded store, as the golden run had; one lookup per
    token and routed expert, src/expert_store.c:72-92): the same layer served
    from a file-backed store reports the same seven numbers, and the same
    outputs."""
    g = golden(f"moe_{case}.npz")
    d, E, k, fe, renorm, gt, ut, dt = (int(v) for v in g["shape"])
    shape = W.MoEShape(case, d, E, k, fe, bool(renorm), gt, ut, dt)
    m = M.DeviceMoE(shape, 1, seed=int(g["seed"][0]))
    gb, ub, db = m.device_layer_bytes(0)
    gs, us, ds = m.slices
    fd, path = tempfile.mkstemp()
    os.unlink(path)
    try:
        os.pwrite(fd, gb.tobytes() + ub.tobytes() + db.tobytes(), 0)
        s = lib.expert_store_create(fd, 0, 1, E)
        for e in range(E):
            sl = _lib.ExpertSlices(e * gs, gb.size + e * us, gb.size + ub.size + e * ds, gs, us, ds)
            lib.expert_store_register(s, 0, e, C.byref(sl))
        m.model.es = s
        xt = torch.from_numpy(g["x"]).to(cuda)
        idx, _ = m.forward(0, xt, torch.from_numpy(g["hb"]).to(cuda), return_routing=True)
        np.testing.assert_array_equal(idx.cpu().numpy(), g["idx"])
        torch.cuda.synchronize()
        st = _lib.ExpertStats()
        lib.expert_store_stats(s, C.byref(st))
        got = [getattr(st, f) for f, _ in _lib.ExpertStats._fields_]
        assert got == [int(v) for v in g["store_stats"]], (got, g["store_stats"])
        lib.expert_store_destroy(s)
    finally:
        os.close(fd)
        m.model.es = m.es
        m.close()


@pytest.mark.parametrize("cap_experts", [0, 2])
def test_truncated_backing_file_is_an_error(cuda, lib, cap_experts):
    """A backing file that ends inside an expert's slices: the lookup that
    must read them returns -EIO (the reference ignores the short read,
    src/expert_store.c:67), and moe_ffn_forward reports it, pinned (unbounded
    store) or paged (a store of two experts)."""
    shape = W.SHAPES["olmoe-q4_k_m"].with_(name="olmoe-8e", E=8)
    m = M.DeviceMoE(shape, 1, seed=67)
    gb, ub, db = m.device_layer_bytes(0)
    gs, us, ds = m.slices
    fd, path = tempfile.mkstemp()
    os.unlink(path)
    try:
        blob = gb.tobytes() + ub.tobytes() + db.tobytes()
        os.pwrite(fd, blob[:len(blob) - ds // 2], 0)  # the last expert's down slice is cut short
        s = lib.expert_store_create(fd, cap_experts * shape.expert_bytes(), 1, shape.E)
        for e in range(shape.E):
            sl = _lib.ExpertSlices(e * gs, gb.size + e * us, gb.size + ub.size + e * ds, gs, us, ds)
            lib.expert_store_register(s, 0, e, C.byref(sl))
        v = _lib.ExpertView()
        assert lib.expert_store_lookup(s, 0, shape.E - 1, C.byref(v)) == -errno.EIO
        assert not v.gate and not v.slot
        assert lib.expert_store_lookup(s, 0, 0, C.byref(v)) == 0  # a whole expert still pages in
        lib.expert_store_release(s, C.byref(v))
        m.model.es = s
        x, hb = W.host_hidden(shape.d, 2, 67)
        xt, hbt = torch.from_numpy(x).to(cuda), torch.from_numpy(hb).to(cuda)
        # top-8 of 8 experts: every token routes to the truncated expert too
        rc = lib.moe_ffn_forward(C.byref(m.model), 0, C.c_void_p(xt.data_ptr()), C.c_void_p(hbt.data_ptr()), 2,
                                 None, None, None)
        assert rc == -errno.EIO
        torch.cuda.synchronize()
        lib.expert_store_destroy(s)
    finally:
        os.close(fd)
        m.model.es = m.es
        m.close()
