import os
import subprocess
import sys

import numpy as np
import pytest
import torch  # noqa: F401  first, so the library binds to the same HIP runtime as torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HERE = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(HERE, "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: full-size parity cases")


def _ensure_built():
    """Build what the tests load when it is absent (a fresh checkout): the
    oracle with make, the HIP library with vireo_amd.build. Where the built
    files are present (the usual case, and always on a GPU machine) nothing
    is rebuilt here."""
    if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "oracle"], check=True,
                       stdout=subprocess.DEVNULL)
    if not os.path.exists(os.path.join(ROOT, "vireo_amd", "libvireo_hip.so")):
        from vireo_amd import build
        build.build()


_ensure_built()


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def lib():
    from vireo_amd import _lib
    return _lib.load()


def golden(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def cuda():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    from vireo_amd import _lib
    _lib.check(_lib.load().vireo_hip_init(0), "vireo_hip_init")
    return torch.device("cuda:0")


def d2h(ptr, nbytes):
    """Copy nbytes at a raw device address to a host uint8 array."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so.7")
    out = np.empty(nbytes, np.uint8)
    rc = hip.hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), C.c_size_t(nbytes), 2)
    assert rc == 0, f"hipMemcpy failed: {rc}"
    return out


def expert_lists(shape, g, u, d):
    """Split stacked expert tensors into per-expert byte arrays."""
    gs, us, ds = shape.slice_bytes()
    E = shape.E
    return ([g[e * gs:(e + 1) * gs] for e in range(E)], [u[e * us:(e + 1) * us] for e in range(E)],
            [d[e * ds:(e + 1) * ds] for e in range(E)])


class RefStoreReplay:
    """The oracle's restatement of the reference's ExpertStore
    (src/expert_store.c), driven by the lookups the reference would make for
    the same work: what expert_store_stats must report. The backing file is a
    sparse temporary file of the model's expert bytes (the oracle pages from
    it; only the counters are compared)."""

    FIELDS = ("requests", "hits", "misses", "bytes_read", "resident_bytes", "capacity_bytes", "experts_resident")

    def __init__(self, oracle, shape, n_layers, capacity, registered=None):
        import tempfile
        self.o, self.E = oracle, shape.E
        gs, us, ds = shape.slice_bytes()
        eb = gs + us + ds
        self.fd, path = tempfile.mkstemp()
        os.unlink(path)
        os.ftruncate(self.fd, n_layers * shape.E * eb)
        self.s = oracle.store_create(self.fd, capacity, n_layers, shape.E)
        for l in range(n_layers):
            for e in range(shape.E):
                if registered is not None and not registered(l, e):
                    continue
                base = (l * shape.E + e) * eb
                oracle.store_register(self.s, l, e, base, base + gs, base + gs + us, gs, us, ds)

    def route(self, layer, idx):
        """moe_ffn's lookups for routing idx [T x k]: token order, selection
        order, each released before the next (src/gguf_run.c:193-213)."""
        for row in np.asarray(idx).reshape(len(idx), -1):
            for e in row:
                rc, view = self.o.store_lookup(self.s, layer, int(e))
                if rc == 0:
                    self.o.store_release(self.s, view)

    def stats(self):
        return dict(zip(self.FIELDS, self.o.store_stats(self.s)))

    def close(self):
        self.o.store_destroy(self.s)
        os.close(self.fd)
