"""The oracle against the reference's own code compiled from source
(oracle/_ref/libvireo_ref.so, built by `make -C oracle ref`) on fresh seeds.
Skipped where that library has not been built (the reference sources are
needed to build it)."""
import numpy as np
import pytest

from conftest import expert_lists
from vireo_amd import workloads as W

pytestmark = pytest.mark.skipif(not __import__("oracle.oracle", fromlist=["Reference"]).Reference.available(),
                                reason="oracle/_ref not built (needs the reference sources)")


@pytest.fixture(scope="module")
def ref():
    from oracle.oracle import Reference
    return Reference()


@pytest.mark.parametrize("typ,n,d", [(W.Q8_0, 2048, 96), (W.Q4_K, 2048, 96), (W.Q6_K, 768, 96), (W.Q5_0, 1024, 40),
                                     (W.F32, 2048, 128)])
def test_matmul_dequant_vs_ref(oracle, ref, typ, n, d):
    for seed in (1, 2):
        if typ == W.F32:
            w = W.host_normal(n * d, seed, 3, sigma=0.02)
        else:
            w = W.host_matrix(typ, n, 0, d, seed, 3)
        x = W.host_normal(n, seed, 4)
        np.testing.assert_array_equal(oracle.matmul(typ, w, x, n, d), ref.matmul(typ, w, x, n, d))
        if typ != W.F32:
            rb = W.row_bytes(typ, n)
            for r in (0, d - 1):
                np.testing.assert_array_equal(oracle.dequant_row(typ, w[r * rb:(r + 1) * rb], n),
                                              ref.dequant_row(typ, w[r * rb:(r + 1) * rb], n))


def test_glue_vs_ref(oracle, ref):
    for seed in range(3):
        v = W.host_normal(4096, seed, 5) * (seed + 1)
        wv = W.host_normal(4096, seed, 6)
        np.testing.assert_array_equal(oracle.rmsnorm(v, wv, 1e-6), ref.rmsnorm(v, wv, 1e-6))
        np.testing.assert_array_equal(oracle.softmax(v[:128]), ref.softmax(v[:128]))
        assert oracle.argmax(v) == ref.argmax(v)


@pytest.mark.parametrize("name,T", [("olmoe-q4_k_m", 3), ("qwen3-30b-a3b-q8_0", 2)])
def test_moe_ffn_vs_ref(oracle, ref, name, T):
    from oracle.oracle import RefMoE
    shape = W.SHAPES[name]
    seed = 31
    router = W.host_router(shape, 0, seed)
    g, u, d = W.host_layer(shape, 0, seed)
    x, hb = W.host_hidden(shape.d, T, seed)
    rm = RefMoE(ref, shape, [router], [g], [u], [d])
    rx, ridx, rprobs = rm.run(0, x, hb)
    rm.close()
    ox, oidx, ow, oprobs = oracle.moe_ffn(shape, router, *expert_lists(shape, g, u, d), x, hb)
    np.testing.assert_array_equal(oidx, ridx)
    np.testing.assert_array_equal(oprobs, rprobs)
    np.testing.assert_array_equal(ox, rx)
