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
