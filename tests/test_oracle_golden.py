"""The oracle against the golden vectors written by the reference's own code
(tests/golden/make_golden.py runs the reference compiled from source).

Every comparison here is bit-exact: the oracle restates the reference's
arithmetic operation for operation.
"""
import hashlib
import os
import tempfile

import numpy as np
import pytest

from conftest import expert_lists, golden
from vireo_amd import workloads as W

KERNEL_TAGS = ["Q8_0_512x16", "Q8_0_96x5", "Q4_K_512x16", "Q6_K_512x16", "Q6_K_768x6", "Q5_0_512x16",
               "F16_100x4", "F32_2048x16"]
TYPE_OF = {"Q8_0": W.Q8_0, "Q4_K": W.Q4_K, "Q6_K": W.Q6_K, "Q5_0": W.Q5_0, "F16": W.F16, "F32": W.F32}


@pytest.fixture(scope="module")
def kernels():
    return golden("kernels.npz")


@pytest.mark.parametrize("tag", KERNEL_TAGS)
def test_matmul_golden(oracle, kernels, tag):
    tname, dims = tag.rsplit("_", 1)
    n, d = map(int, dims.split("x"))
    typ = TYPE_OF[tname]
    w, x = kernels[f"{tag}_w"], kernels[f"{tag}_x"]
    y = oracle.matmul(typ, w.view(np.uint8) if typ != W.F32 else w, x, n, d)
    np.testing.assert_array_equal(y, kernels[f"{tag}_y"])
    if f"{tag}_deq" in kernels:
        wb = w.view(np.uint8).reshape(-1)
        rb = wb.size // d
        deq = np.stack([oracle.dequant_row(typ, wb[i * rb:(i + 1) * rb], n) for i in range(d)])
        np.testing.assert_array_equal(deq, kernels[f"{tag}_deq"])


def test_glue_golden(oracle, kernels):
    np.testing.assert_array_equal(oracle.rmsnorm(kernels["rmsnorm_x"], np.ones(2048, np.float32), 1e-6),
                                  kernels["rmsnorm_y"])
    np.testing.assert_array_equal(oracle.softmax(kernels["softmax_x"]), kernels["softmax_y"])
    assert oracle.argmax(kernels["argmax_x"]) == int(kernels["argmax_y"][0])


def _shape(g):
    d, E, k, fe, renorm, gt, ut, dt = (int(v) for v in g["shape"])
    return W.MoEShape("golden", d, E, k, fe, bool(renorm), gt, ut, dt)


@pytest.mark.parametrize("case", ["tiny_q4km", "tiny_q8", "olmoe_q8_0", "qwen3_q4_k_m"])
def test_moe_ffn_golden(oracle, case):
    g = golden(f"moe_{case}.npz")
    shape = _shape(g)
    seed = int(g["seed"][0])
    router = W.host_router(shape, 0, seed)
    gt, ut, dt = W.host_layer(shape, 0, seed)
    h = hashlib.sha256()
    for a in (router, gt, ut, dt):
        h.update(np.ascontiguousarray(a).tobytes())
    assert h.hexdigest() == str(g["weights_sha256"]), "synthetic generator changed: regenerate the fixtures"
    G, U, D = expert_lists(shape, gt, ut, dt)
    xo, idx, w, probs = oracle.moe_ffn(shape, router, G, U, D, g["x"], g["hb"])
    np.testing.assert_array_equal(idx, g["idx"])
    np.testing.assert_array_equal(probs, g["probs"])
    np.testing.assert_array_equal(xo, g["x_out"])


def test_store_golden(oracle):
    """The reference unit test's scenario through the restated pager: bytes
    correct, budget respected, leased expert survives, stats as the reference
    printed them (requests=125 hits=0 misses=125 read=1000KB resident=80KB/80KB)."""
    import ctypes as C
    g = golden("store.npz")
    NL, NE, capn = (int(v) for v in g["dims"])
    SZ = [int(v) for v in g["sizes"]]
    fd, path = tempfile.mkstemp()
    os.unlink(path)
    try:
        locs, off = [], 0
        for l in range(NL):
            for e in range(NE):
                loc = []
                for s, n in enumerate(SZ):
                    os.pwrite(fd, ((l * 131 + e * 17 + s * 7 + np.arange(n)) & 0xFF).astype(np.uint8).tobytes(), off)
                    loc.append(off)
                    off += n
                locs.append(loc)
        st = oracle.store_create(fd, sum(SZ) * capn, NL, NE)
        for l in range(NL):
            for e in range(NE):
                oracle.store_register(st, l, e, *locs[l * NE + e], *SZ)
        for l in range(NL):
            for e in range(NE):
                rc, view = oracle.store_lookup(st, l, e)
                assert rc == 0
                for s, n in enumerate(SZ):
                    got = np.ctypeslib.as_array(C.cast(view[s], C.POINTER(C.c_uint8)), (n,))
                    np.testing.assert_array_equal(got, ((l * 131 + e * 17 + s * 7 + np.arange(n)) & 0xFF))
                oracle.store_release(st, view)
        assert oracle.store_stats(st) == [int(v) for v in g["after_sweep"]]
        rc, pinned = oracle.store_lookup(st, 0, 0)
        for l in range(NL):
            for e in range(1, NE):
                rc, view = oracle.store_lookup(st, l, e)
                if rc == 0:
                    oracle.store_release(st, view)
        got = np.ctypeslib.as_array(C.cast(pinned[0], C.POINTER(C.c_uint8)), (SZ[0],))
        np.testing.assert_array_equal(got, (np.arange(SZ[0]) & 0xFF))
        oracle.store_release(st, pinned)
        stats = oracle.store_stats(st)
        assert stats == [int(v) for v in g["after_flood"]]
        assert stats[:4] == [125, 0, 125, 1000 * 1024] and stats[4] == stats[5] == 80 * 1024
        oracle.store_destroy(st)
    finally:
        os.close(fd)
