"""moe_ffn_forward_noalloc: the entry point for callers that cannot allocate
(its workspace is a fixed static device region). Its results equal
moe_ffn_forward's bit for bit on the same inputs (the same kernels run), on
consecutive calls whose second is smaller than the first, on every plan it
takes (matrix-core GEMMs on GGUF rows and on packed Q8_0 fragments, the
matrix-core decode batch on packed tiles, register-input groups, the decode
plan for a batch of tokens and for one token);
it refuses calls whose intermediates exceed the region (-E2BIG) and layers
that are not pinned yet (-EINVAL), and it allocates no device memory."""
import ctypes as C
import errno

import numpy as np
import pytest
import torch

from vireo_amd import _lib
from vireo_amd import moe as M
from vireo_amd import workloads as W

pytestmark = pytest.mark.gpu


def _call(lib, fn, m, layer, x, hb, T, idx, w):
    return fn(C.byref(m.model), layer, C.c_void_p(x.data_ptr()), C.c_void_p(hb.data_ptr()), T,
              C.c_void_p(idx.data_ptr()), C.c_void_p(w.data_ptr()), None)


def _check_noalloc(cuda, lib, m, shape, sizes, seed, unpinned, too_big):
    """Runs `sizes` ((layer, tokens), each call no larger than the one before)
    through moe_ffn_forward, then through moe_ffn_forward_noalloc: the same
    bits, no device memory allocated. `unpinned` (layer, tokens) is refused
    while its layer is not pinned; `too_big` tokens exceed the region."""
    inputs = {}
    for layer, T in sizes:
        x, hb = W.host_hidden(shape.d, T, seed + T)
        inputs[(layer, T)] = (x, torch.from_numpy(hb).to(cuda))
    # refused before the layer is pinned: pinning allocates
    x0, hb0 = inputs[unpinned]
    T0 = unpinned[1]
    xg = torch.from_numpy(x0).to(cuda)
    idx = torch.empty((T0, shape.k), dtype=torch.int32, device=cuda)
    w = torch.empty((T0, shape.k), dtype=torch.float32, device=cuda)
    assert _call(lib, lib.moe_ffn_forward_noalloc, m, unpinned[0], xg, hb0, T0, idx, w) == -errno.EINVAL
    # the reference results (this also pins the layers and makes their packed copies)
    want = {}
    for layer, T in sizes:
        x, hb = inputs[(layer, T)]
        xr = torch.from_numpy(x).to(cuda)
        ir = torch.empty((T, shape.k), dtype=torch.int32, device=cuda)
        wr = torch.empty((T, shape.k), dtype=torch.float32, device=cuda)
        _lib.check(_call(lib, lib.moe_ffn_forward, m, layer, xr, hb, T, ir, wr), "moe_ffn_forward")
        want[(layer, T)] = (xr.cpu().numpy(), ir.cpu().numpy(), wr.cpu().numpy())
    outs = {}
    for layer, T in sizes:
        x, hb = inputs[(layer, T)]
        outs[(layer, T)] = (torch.from_numpy(x).to(cuda), torch.empty((T, shape.k), dtype=torch.int32, device=cuda),
                            torch.empty((T, shape.k), dtype=torch.float32, device=cuda))
    big_x = torch.zeros((too_big, shape.d), dtype=torch.float32, device=cuda)
    big_i = torch.empty((too_big, shape.k), dtype=torch.int32, device=cuda)
    big_w = torch.empty((too_big, shape.k), dtype=torch.float32, device=cuda)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for layer, T in sizes:
        x, hb = inputs[(layer, T)]
        xo, io, wo = outs[(layer, T)]
        _lib.check(_call(lib, lib.moe_ffn_forward_noalloc, m, layer, xo, hb, T, io, wo), "moe_ffn_forward_noalloc")
    # a call whose intermediates exceed the fixed region
    assert _call(lib, lib.moe_ffn_forward_noalloc, m, 0, big_x, big_x, too_big, big_i, big_w) == -errno.E2BIG
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0, "device memory was allocated"
    for key, (xo, io, wo) in outs.items():
        xw, iw, ww = want[key]
        np.testing.assert_array_equal(io.cpu().numpy(), iw, err_msg=str(key))
        np.testing.assert_array_equal(wo.cpu().numpy(), ww, err_msg=str(key))
        np.testing.assert_array_equal(xo.cpu().numpy(), xw, err_msg=str(key))


def test_noalloc_matches_moe_ffn_forward(cuda, lib):
    """Q4_K_M experts: the matrix-core GEMMs (96 tokens), the matrix-core
    decode batch on its packed 16-row tiles (40 and 5), the decode plan for
    a batch of 3 tokens and the one-token plan."""
    shape = W.SHAPES["qwen3-30b-a3b-q4_k_m"]
    m = M.DeviceMoE(shape, 2, seed=91)
    try:
        _check_noalloc(cuda, lib, m, shape, [(0, 96), (1, 40), (1, 5), (1, 3), (0, 1), (1, 1)], 91, (1, 5), 2048)
    finally:
        m.close()


def test_noalloc_q8_fragments(cuda, lib):
    """Q8_0 experts: calls of 64+ tokens on the matrix-core GEMMs reading the
    packed operand fragments the first moe_ffn_forward made, 20 tokens on the
    register-input groups and 6 on the decode plan for a batch."""
    shape = W.SHAPES["olmoe-q8_0"]
    m = M.DeviceMoE(shape, 1, seed=93)
    try:
        _check_noalloc(cuda, lib, m, shape, [(0, 130), (0, 70), (0, 20), (0, 6)], 93, (0, 70), 2048)
    finally:
        m.close()
