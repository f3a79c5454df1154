"""The C boundary as a C program sees it: include/*.h compiled by gcc, the
library linked with -lvireo_hip (what a maintainer adds to the reference's
Makefile), the reference's own headers and ExpertStore beside it."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CDIR = os.path.join(ROOT, "tests", "c")
LIBDIR = os.path.join(ROOT, "vireo_amd")
REF_SRC = "/root/reference/src"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
CFLAGS = ["-std=c11", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
          "-I", os.path.join(ROCM, "include")]
LDFLAGS = ["-L", LIBDIR, "-lvireo_hip", f"-Wl,-rpath,{LIBDIR}", "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
           f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"]


def gcc(args, tmp_path):
    r = subprocess.run(["gcc", *args], capture_output=True, text=True, cwd=tmp_path)
    assert r.returncode == 0, r.stdout + r.stderr


def test_caller_compiles_and_links(tmp_path):
    exe = str(tmp_path / "moe_caller")
    gcc([*CFLAGS, os.path.join(CDIR, "moe_caller.c"), "-o", exe, *LDFLAGS], tmp_path)
    assert os.path.exists(exe)


def test_library_binds_its_own_symbols():
    """Linked with -Bsymbolic: the library's calls to expert_store_* stay on
    its own definitions even when an executable defines the same names."""
    r = subprocess.run(["readelf", "-d", os.path.join(LIBDIR, "libvireo_hip.so")], capture_output=True, text=True)
    assert r.returncode == 0
    assert "SYMBOLIC" in r.stdout


@pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="reference sources not mounted")
@pytest.mark.parametrize("ref_first", [True, False])
def test_headers_with_reference_headers(tmp_path, ref_first):
    args = [*CFLAGS, "-Wno-unused-function", "-I", REF_SRC, "-c", os.path.join(CDIR, "include_order.c"),
            "-o", str(tmp_path / "io.o")]
    if ref_first:
        args.insert(0, "-DREF_FIRST")
    gcc(args, tmp_path)


@pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="reference sources not mounted")
def test_foreign_store_refused(tmp_path):
    """A program that still links the reference's CPU ExpertStore gets
    -EINVAL from the GPU entry points for that store (no device call made)."""
    exe = str(tmp_path / "foreign")
    gcc([*CFLAGS, "-I", REF_SRC, os.path.join(CDIR, "foreign_store.c"), os.path.join(REF_SRC, "expert_store.c"),
         "-o", exe, *LDFLAGS], tmp_path)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.gpu
def test_c_caller_runs_against_oracle(cuda, oracle, tmp_path):
    """tests/c/moe_caller.c on a synthetic GGUF MoE file: every layer's
    moe_ffn_forward from C (synchronous, stream NULL) and one stack step
    match the oracle on the bytes written into the file."""
    import numpy as np
    from conftest import expert_lists
    from vireo_amd import gguf as G
    from vireo_amd import workloads as W
    exe = str(tmp_path / "moe_caller")
    gcc([*CFLAGS, os.path.join(CDIR, "moe_caller.c"), "-o", exe, *LDFLAGS], tmp_path)
    shape = W.SHAPES["qwen3-30b-a3b-q4_k_m"].with_(name="qwen3-16e", E=16)
    L, vocab = 3, 512
    path = str(tmp_path / "m.gguf")
    arr = G.write_moe_gguf(path, shape, L, seed=83, vocab=vocab)
    x, xb = W.host_hidden(shape.d, 1, 83)
    x, xb = x[0], xb[0]
    x.tofile(str(tmp_path / "x.bin"))
    xb.tofile(str(tmp_path / "xb.bin"))
    r = subprocess.run([exe, path, str(tmp_path / "x.bin"), str(tmp_path / "xb.bin"), str(tmp_path / "out.bin")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    out = np.fromfile(str(tmp_path / "out.bin"), np.float32)
    d = shape.d
    xo = x.copy()
    layers = [expert_lists(shape, *arr["experts"][l]) for l in range(L)]
    for l in range(L):
        xo = oracle.moe_ffn(shape, arr["routers"][l], *layers[l], xo[None], xb[None])[0][0]
        got = out[:d] if l == 0 else out[d:2 * d]
        if l in (0, L - 1):
            rel = np.abs((got - x) - (xo - x)).max() / np.abs(xo - x).max()
            assert rel <= 2e-3, (l, rel)
    # the stack step from token 3 (tied or untied head as written)
    rb = W.row_bytes(W.Q8_0, d)
    emb, head = arr["token_embd"], arr["output"]
    xs = oracle.dequant_row(W.Q8_0, emb[3 * rb:4 * rb], d)
    for l in range(L):
        xs = oracle.moe_ffn(shape, arr["routers"][l], *layers[l], xs[None],
                            oracle.rmsnorm(xs, arr["ffn_norm"][l], W.EPS)[None])[0][0]
    logits = oracle.matmul(W.Q8_0, head, oracle.rmsnorm(xs, arr["out_norm"], W.EPS), d, vocab)
    top2 = np.sort(logits)[-2:]
    if top2[1] - top2[0] > 2e-3 * np.abs(logits).max():
        assert int(out[2 * d]) == oracle.argmax(logits)
    print(r.stdout.strip())
