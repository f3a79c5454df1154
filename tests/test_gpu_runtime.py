"""Library runtime behaviour on the GPU: graphs captured before the library
grows its buffers keep working, and a fused grid-wide wait that gives up is
reported (the poll limit forced to 0 from the host, so no wave ever waits)."""
import ctypes as C
import errno

import numpy as np
import pytest
import torch

from vireo_amd import _lib
from vireo_amd import moe as M
from vireo_amd import stack as S
from vireo_amd import workloads as W

pytestmark = pytest.mark.gpu


def test_graph_survives_workspace_growth(cuda, lib):
    """Capture single-token decode steps in a HIP graph, then run a call
    large enough to grow the per-device workspace (a 512-token prefill),
    then replay: the replays must still equal the eager steps (the graph
    keeps the buffers it captured; they are not freed on growth)."""
    shape = W.SHAPES["qwen3-30b-a3b-q4_k_m"]
    m = M.DeviceMoE(shape, 2, seed=71)
    n = 6
    x0, hb0 = W.host_hidden(shape.d, n, 71)
    hb = torch.from_numpy(hb0).to(cuda)
    xe = torch.from_numpy(x0).to(cuda)
    for i in range(n):  # eager reference (also pins both layers and sizes the decode workspace)
        m.forward(i % 2, xe[i:i + 1], hb[i:i + 1])
    torch.cuda.synchronize()
    xg = torch.from_numpy(x0).to(cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(n):
            m.forward(i % 2, xg[i:i + 1], hb[i:i + 1], stream=s)
    torch.cuda.synchronize()
    # a larger call: the workspace grows to a new allocation
    xp, hp = (torch.from_numpy(a).to(cuda) for a in W.host_hidden(shape.d, 512, 72))
    m.forward(0, xp, hp)
    torch.cuda.synchronize()
    for rep in range(3):
        xg.copy_(torch.from_numpy(x0))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(xg, xe), f"replay {rep} differs from the eager steps"
        m.forward(1, xp[:64], hp[:64])  # eager work between replays
        torch.cuda.synchronize()
    m.close()


@pytest.mark.parametrize("plan", [3, 5])
def test_fused_wait_timeout_is_reported(cuda, lib, plan):
    """Plan 3 (one fused experts kernel whose workgroups meet once) and plan 5
    (the whole layer in one launch, meeting twice): with the
    poll limit at 0 every workgroup gives up at once, the kernel still ends,
    a synchronous call returns -ETIMEDOUT and a stream call's status reads
    -ETIMEDOUT; with the default limit the same call succeeds and equals the
    separate-kernel plan."""
    shape = W.SHAPES["qwen3-30b-a3b-q4_k_m"]
    m = M.DeviceMoE(shape, 1, seed=73)
    x0, hb0 = W.host_hidden(shape.d, 1, 73)
    hb = torch.from_numpy(hb0).to(cuda)
    ref = torch.from_numpy(x0).to(cuda)
    m.forward(0, ref, hb)  # plan 0 (separate kernels)
    torch.cuda.synchronize()
    _lib.check(lib.vireo_hip_set_path(plan), "set_path")
    try:
        assert lib.vireo_hip_status(None) == 0
        _lib.check(lib.vireo_hip_set_spin_limit(0), "set_spin_limit")
        x = torch.from_numpy(x0).to(cuda)
        torch.cuda.synchronize()
        rc = lib.moe_ffn_forward(C.byref(m.model), 0, C.c_void_p(x.data_ptr()), C.c_void_p(hb.data_ptr()), 1,
                                 None, None, None)
        assert rc == -errno.ETIMEDOUT
        assert lib.vireo_hip_status(None) == 0  # the synchronous call read and cleared it
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        m.forward(0, x, hb, stream=st)  # on a stream: only enqueued, so the status reports it
        assert lib.vireo_hip_status(M._stream_handle(st)) == -errno.ETIMEDOUT
        assert lib.vireo_hip_status(None) == 0
        _lib.check(lib.vireo_hip_set_spin_limit(1 << 18), "set_spin_limit")
        x = torch.from_numpy(x0).to(cuda)
        torch.cuda.synchronize()
        rc = lib.moe_ffn_forward(C.byref(m.model), 0, C.c_void_p(x.data_ptr()), C.c_void_p(hb.data_ptr()), 1,
                                 None, None, None)
        assert rc == 0
        assert torch.equal(x, ref)
    finally:
        lib.vireo_hip_set_spin_limit(1 << 18)
        lib.vireo_hip_set_path(0)
        m.close()


@pytest.mark.parametrize("plan", [3, 5])
def test_stack_step_wait_timeout_is_reported(cuda, lib, plan):
    """A synchronous moe_stack_step under a plan whose workgroups wait for
    each other returns -ETIMEDOUT when the waits give up (poll limit 0), and
    the status word is left clear; with the default limit the same step
    succeeds and picks the plan-0 step's token."""
    st = S.DeviceStack(W.SHAPES["qwen3-30b-a3b-q4_k_m"], 2, vocab=512, seed=79)
    token = torch.tensor([7], dtype=torch.int32, device=cuda)
    try:
        st.step(token)  # plan 0
        want = int(token.item())
        _lib.check(lib.vireo_hip_set_path(plan), "set_path")
        assert lib.vireo_hip_status(None) == 0
        _lib.check(lib.vireo_hip_set_spin_limit(0), "set_spin_limit")
        token.fill_(7)
        torch.cuda.synchronize()
        rc = lib.moe_stack_step(C.byref(st.st), M._ptr(token), M._ptr(st.x), M._ptr(st.xb), M._ptr(st.logits), None)
        assert rc == -errno.ETIMEDOUT
        assert lib.vireo_hip_status(None) == 0
        _lib.check(lib.vireo_hip_set_spin_limit(1 << 18), "set_spin_limit")
        token.fill_(7)
        st.step(token)
        assert int(token.item()) == want
    finally:
        lib.vireo_hip_set_spin_limit(1 << 18)
        lib.vireo_hip_set_path(0)
        st.close()
