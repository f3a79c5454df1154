"""qmatvec / qdequant_rows / rmsnorm / argmax on the GPU against the oracle,
the golden vectors and the rigorous error bound of an fp32 dot product."""
import ctypes as C

import numpy as np
import pytest
import torch

import qformats as Q
from conftest import golden
from vireo_amd import moe as M
from vireo_amd import workloads as W

pytestmark = pytest.mark.gpu
U24 = 2.0 ** -24

CASES = [(W.Q8_0, 2048, 768), (W.Q8_0, 96, 33), (W.Q4_K, 2048, 768), (W.Q6_K, 768, 2048), (W.Q6_K, 1024, 37),
         (W.Q5_0, 1024, 64), (W.F16, 300, 16), (W.F32, 2048, 128), (W.Q4_K, 256, 1),
         # register-input kernel, two rows per wave (1024 to 8191 rows of 32 to 128 items)
         (W.Q4_K, 4096, 2048), (W.Q6_K, 2048, 1536), (W.Q8_0, 2048, 1025)]


def _weights(typ, n, d, seed):
    if typ == W.F32:
        return W.host_normal(n * d, seed, 3, sigma=0.02).view(np.uint8)
    if typ == W.F16:
        return W.host_normal(n * d, seed, 3).astype(np.float16).view(np.uint8)
    return W.host_matrix(typ, n, 0, d, seed, 3)


@pytest.mark.parametrize("typ,n,d", CASES)
def test_qmatvec(cuda, oracle, typ, n, d):
    w = _weights(typ, n, d, seed=n + d)
    x = W.host_normal(n, 5, 6)
    wt = torch.from_numpy(w).to(cuda)
    y = torch.empty(d, dtype=torch.float32, device=cuda)
    M.qmatvec(y, torch.from_numpy(x).to(cuda), wt, typ, n, d)
    yg = y.cpu().numpy().astype(np.float64)
    wd = Q.decode(typ, w, n).astype(np.float64)
    exact = wd @ x.astype(np.float64)
    bound = (n + 2) * U24 * (np.abs(wd) @ np.abs(x.astype(np.float64))) + 1e-30
    assert np.all(np.abs(yg - exact) <= bound)
    yo = oracle.matmul(typ, w if typ != W.F32 else w.view(np.float32), x, n, d)
    assert np.abs(yg - yo).max() <= 2e-3 * np.abs(yo).max()


@pytest.mark.parametrize("typ,n,rows", [(W.Q8_0, 2048, 16), (W.Q4_K, 2048, 16), (W.Q6_K, 768, 16), (W.Q5_0, 512, 8),
                                        (W.F16, 300, 4), (W.F32, 64, 4)])
def test_dequant_bit_exact(cuda, oracle, typ, n, rows):
    w = _weights(typ, n, rows, seed=11)
    out = M.dequant_rows(typ, torch.from_numpy(w).to(cuda), n, rows).cpu().numpy()
    rb = w.size // rows
    want = np.stack([oracle.dequant_row(typ, w[i * rb:(i + 1) * rb], n) for i in range(rows)])
    np.testing.assert_array_equal(out, want)


def test_golden_kernels_on_gpu(cuda):
    g = golden("kernels.npz")
    for tag in ("Q8_0_512x16", "Q8_0_96x5", "Q4_K_512x16", "Q6_K_512x16", "Q6_K_768x6", "Q5_0_512x16"):
        tname, dims = tag.rsplit("_", 1)
        n, d = map(int, dims.split("x"))
        typ = {"Q8_0": W.Q8_0, "Q4_K": W.Q4_K, "Q6_K": W.Q6_K, "Q5_0": W.Q5_0}[tname]
        wt = torch.from_numpy(g[f"{tag}_w"].view(np.uint8)).to(cuda)
        np.testing.assert_array_equal(M.dequant_rows(typ, wt, n, d).cpu().numpy(), g[f"{tag}_deq"])
        y = torch.empty(d, dtype=torch.float32, device=cuda)
        M.qmatvec(y, torch.from_numpy(g[f"{tag}_x"]).to(cuda), wt, typ, n, d)
        want = g[f"{tag}_y"]
        assert np.abs(y.cpu().numpy() - want).max() <= 2e-3 * np.abs(want).max()


def test_rmsnorm(cuda, oracle):
    x = W.host_normal(4 * 2048, 1, 1).reshape(4, 2048) * np.float32(3)
    w = W.host_normal(2048, 2, 2)
    out = M.rmsnorm(torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda), 1e-6).cpu().numpy()
    for r in range(4):
        np.testing.assert_allclose(out[r], oracle.rmsnorm(x[r], w, 1e-6), rtol=2e-5, atol=1e-6)


@pytest.mark.parametrize("n", [2048, 768, 5, 20000])
def test_rmsnorm_exact(cuda, oracle, n):
    """vireo_rmsnorm_exact equals the reference's rmsnorm bit for bit (its
    in-order fp32 sum of squares), with an F32 weight row and with none; rows
    longer than its LDS buffer (20000) sum from the output row."""
    from vireo_amd import _lib
    lib = _lib.load()
    x = W.host_normal(n, 3, 3) * np.float32(7)
    x[::97] *= np.float32(1e-3)  # magnitudes that make the order of the sum matter
    for w in (W.host_normal(n, 4, 4), None):
        xt = torch.from_numpy(x).to(cuda)
        o = torch.empty_like(xt)
        wt = torch.from_numpy(w).to(cuda) if w is not None else None
        _lib.check(lib.vireo_rmsnorm_exact(C.c_void_p(o.data_ptr()), C.c_void_p(xt.data_ptr()),
                                           C.c_void_p(wt.data_ptr()) if wt is not None else None, n,
                                           C.c_float(1e-6), None), "vireo_rmsnorm_exact")
        want = oracle.rmsnorm(x, w if w is not None else np.ones(n, np.float32), 1e-6)
        np.testing.assert_array_equal(o.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n,ties", [(151936, (7, 100000)), (151936, (4096 * 3 - 1, 4096 * 3, 151935)),
                                    (151936, (151935,)), (5, (0, 4)), (1, (0,)), (4097, (4096,))])
def test_argmax_first_max(cuda, oracle, n, ties):
    """The first index of the maximum, as the reference's strict '>' scan:
    ties inside a chunk, across the two-launch reduction's chunk boundaries,
    at the last element, and a single element."""
    v = W.host_normal(n, 3, 3)
    top = v.max() + 1
    for t in ties:
        v[t] = top
    got = int(M.argmax(torch.from_numpy(v).to(cuda)).cpu()[0])
    assert got == min(ties) == oracle.argmax(v)


@pytest.mark.parametrize("typ,n,d", [(W.Q8_0, 2048, 8197), (W.Q4_K, 2048, 4096), (W.Q6_K, 2048, 4100),
                                     (W.Q8_0, 4096, 4099), (W.Q8_0, 1056, 5000), (W.Q6_K, 3072, 4096)])
def test_qmatvec_many_rows(cuda, oracle, typ, n, d):
    """Matrices with many rows (the LM head's path: inputs kept in registers,
    8 rows fetched per wave at a time): one or two items per lane, row
    counts that leave a partial last batch, item counts that leave lanes
    idle; against the oracle's gguf_matmul within 2e-3 of the largest output."""
    w = W.host_matrix(typ, n, 0, d, 71, W.stream_id(0, W.KIND_LM_HEAD))
    x = W.host_normal(n, 72, 1)
    y = torch.empty(d, dtype=torch.float32, device=cuda)
    M.qmatvec(y, torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda), typ, n, d)
    want = oracle.matmul(typ, w, x, n, d)
    assert np.abs(y.cpu().numpy() - want).max() <= 2e-3 * np.abs(want).max()


# binary16 scales that exercise every branch of gguf_f16_to_f32 (src/gguf_compute.c:17-36):
# zero and negative zero, the smallest and largest subnormals, the smallest normal, the largest
# finite value, both infinities, quiet and signalling NaNs
SPECIAL_F16 = [0x0000, 0x8000, 0x0001, 0x83FF, 0x03FF, 0x0400, 0x7BFF, 0x7C00, 0xFC00, 0x7E00, 0x7C01, 0xFD55]


@pytest.mark.parametrize("typ,n", [(W.Q8_0, 256), (W.Q4_K, 512), (W.Q6_K, 512)])
def test_dequant_special_scales(cuda, oracle, typ, n):
    """Blocks whose fp16 scales (d, and dmin for Q4_K) are subnormal, infinite
    or NaN dequantize on the GPU to the reference's values: bit-equal where
    finite, the same infinities and NaN in the same places (products of inf
    and a zero quant are NaN in both)."""
    rows = len(SPECIAL_F16)
    w = _weights(typ, n, rows, seed=13).copy()
    rb = w.size // rows
    bb = {W.Q8_0: 34, W.Q4_K: 144, W.Q6_K: 210}[typ]
    for r, h in enumerate(SPECIAL_F16):
        for b in range(rb // bb):
            blk = r * rb + b * bb
            hb = np.array([h], np.uint16).view(np.uint8)
            if typ == W.Q8_0:
                w[blk:blk + 2] = hb
            elif typ == W.Q4_K:  # d, then dmin (the special value with another one beside it)
                w[blk:blk + 2] = hb
                w[blk + 2:blk + 4] = np.array([SPECIAL_F16[(r + b + 3) % rows]], np.uint16).view(np.uint8)
            else:  # Q6_K: d is the last two bytes of the block
                w[blk + 208:blk + 210] = hb
    out = M.dequant_rows(typ, torch.from_numpy(w).to(cuda), n, rows).cpu().numpy()
    want = np.stack([oracle.dequant_row(typ, w[i * rb:(i + 1) * rb], n) for i in range(rows)])
    np.testing.assert_array_equal(np.isnan(out), np.isnan(want))
    fin = ~np.isnan(want)
    np.testing.assert_array_equal(out[fin], want[fin])
    assert np.isinf(want).any() and np.isnan(want).any()
