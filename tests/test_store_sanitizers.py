"""The HBM ExpertStore (vireo_amd/csrc/expert_store.c) under ThreadSanitizer
and under AddressSanitizer + UndefinedBehaviorSanitizer, on the CPU.

tests/c/store_race.c drives a file-backed store smaller than the model the
way the paged MoE plan does (page-ins on a copy stream through the parallel
pread workers and the pinned staging ring, a copy fence, stream-ordered reads
of every byte of each view, leases dropped behind them, read-ahead of the
next layer's guess, routing notes copied back, synchronous lookups between),
linked against tests/c/hip_host_stub.c, which runs each stream's work on a
thread of its own over host memory. Bar: every byte read equals the file and
the sanitizers report nothing. Removing the store's wait on a reused block's
event (page_in's hipStreamWaitEvent) makes ThreadSanitizer report the copy
into the block racing with the previous owner's reads."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SOURCES = [os.path.join(ROOT, "tests", "c", "store_race.c"), os.path.join(ROOT, "tests", "c", "hip_host_stub.c"),
           os.path.join(ROOT, "vireo_amd", "csrc", "expert_store.c")]
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


@pytest.mark.parametrize("sanitizer", ["thread", "address,undefined"])
def test_expert_store_under_sanitizer(tmp_path, sanitizer):
    exe = str(tmp_path / "store_race")
    cmd = ["gcc", "-std=c11", "-D_GNU_SOURCE", "-D__HIP_PLATFORM_AMD__", "-O1", "-g", "-fno-omit-frame-pointer",
           f"-fsanitize={sanitizer}", "-fno-sanitize-recover=all", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(ROCM, "include"), *SOURCES, "-o", exe, "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and "sanitize" in r.stderr and ("cannot find" in r.stderr or "unrecognized" in r.stderr):
        pytest.skip(f"gcc has no -fsanitize={sanitizer} runtime here")
    assert r.returncode == 0, r.stderr
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1", ASAN_OPTIONS="detect_leaks=1:halt_on_error=1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "every byte read matched" in out
    assert "Sanitizer" not in out, out[-4000:]
