"""The synthetic workload generator on the host: counter-based determinism,
the distribution of the draws, and the quantizers' round-trip error."""
import ctypes as C

import numpy as np
import pytest

import qformats as Q
from vireo_amd import workloads as W


def test_normal_is_counter_based():
    a = W.host_normal(10000, seed=9, stream=3)
    b = W.host_normal(4000, seed=9, stream=3, first=6000)
    np.testing.assert_array_equal(a[6000:], b)
    assert not np.array_equal(a, W.host_normal(10000, seed=9, stream=4))
    assert not np.array_equal(a, W.host_normal(10000, seed=10, stream=3))


def test_normal_moments():
    v = W.host_normal(1 << 20, seed=1, stream=1).astype(np.float64)
    assert abs(v.mean()) < 5e-3 and abs(v.std() - 1) < 5e-3
    assert abs(((v - v.mean()) ** 3).mean()) < 2e-2       # symmetric
    assert abs((v ** 4).mean() / v.var() ** 2 - 3) < 5e-2  # normal kurtosis
    s = W.host_normal(1000, seed=1, stream=1, sigma=0.02)
    np.testing.assert_allclose(s, (v[:1000] * 0.02).astype(np.float32), rtol=1e-6)


def test_matrix_rows_are_a_slice_of_the_stack():
    full = W.host_matrix(W.Q4_K, 512, 0, 12, seed=5, stream=2)
    rb = W.row_bytes(W.Q4_K, 512)
    part = W.host_matrix(W.Q4_K, 512, 7, 3, seed=5, stream=2)
    np.testing.assert_array_equal(full[7 * rb:10 * rb], part)


def _quantize(lib, typ, v, n):
    rows = v.size // n
    dst = np.zeros(rows * W.row_bytes(typ, n), np.uint8)
    assert lib.vireo_quantize(typ, v.ctypes.data_as(C.c_void_p), dst.ctypes.data_as(C.c_void_p), n, rows) == 0
    return dst


@pytest.mark.parametrize("typ,tol", [(W.Q8_0, 0.0068), (W.Q6_K, 0.024), (W.Q5_0, 0.056), (W.Q4_K, 0.098)])
def test_quantizer_round_trip(lib, typ, tol):
    """RMS error of N(0, 0.02) data within 1.25x of step/sqrt(12) for the
    format's block range (8, 6, 5 and 4 bits per weight)."""
    v = W.host_normal(64 * 512, seed=3, stream=7, sigma=0.02)
    deq = Q.decode(typ, _quantize(lib, typ, v, 512), 512).reshape(-1)
    rel = np.sqrt(((deq - v) ** 2).mean() / (v ** 2).mean())
    assert rel < tol
    np.testing.assert_array_equal(np.sign(deq[np.abs(v) > 0.03]), np.sign(v[np.abs(v) > 0.03]))


def test_q8_0_exact_grid(lib):
    """Values on the Q8_0 grid q * 2^-4 with amax = 127 * 2^-4 round-trip exactly."""
    rng = np.random.default_rng(0)
    q = rng.integers(-127, 128, size=(16, 32))
    q[:, 0] = 127
    v = (q * 2.0 ** -4).astype(np.float32).reshape(-1)
    np.testing.assert_array_equal(Q.decode(W.Q8_0, _quantize(lib, W.Q8_0, v, 32), 32).reshape(-1), v)


def test_f16_f32_quantize_are_conversions(lib):
    v = W.host_normal(256, seed=1, stream=1)
    np.testing.assert_array_equal(_quantize(lib, W.F32, v, 256).view(np.float32), v)
    np.testing.assert_array_equal(_quantize(lib, W.F16, v, 256).view(np.float16), v.astype(np.float16))


def test_hidden_is_rmsnormed():
    x, hb = W.host_hidden(2048, 4, seed=2)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + W.EPS)
    np.testing.assert_allclose(hb, want, rtol=3e-6)
    np.testing.assert_array_equal(x[0], W.host_normal(2048, 2, W.stream_id(0, W.KIND_HIDDEN)))


def test_zipf_bias():
    b = W.zipf_bias(128, 1.1, seed=0).astype(np.float64)
    p = np.sort(np.exp(b))[::-1]
    assert abs(p.sum() - 1) < 1e-5
    np.testing.assert_allclose(p[0] / p[1:6], (np.arange(2, 7)) ** 1.1, rtol=1e-5)
    assert np.array_equal(W.zipf_bias(128, 1.1, 0), W.zipf_bias(128, 1.1, 0))
