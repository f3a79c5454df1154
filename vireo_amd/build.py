"""Build the vireo-hip shared library in-tree for gfx950.

Every .hip file under csrc/ is compiled by hipcc (device code for gfx950 with
packed-FP32 instructions disabled), every .c file by gcc against the HIP
runtime headers, and the objects are linked into vireo_amd/libvireo_hip.so.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libvireo_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the first kernel arguments arrive in SGPRs at wave launch instead of
    # through a scalar load (gfx950 kernarg preloading)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-I", INCLUDE, "-I", CSRC,
]
C_FLAGS = ["-O2", "-fPIC", "-std=c11", "-pthread", "-Wall", "-Wextra", "-I", INCLUDE, "-I", os.path.join(ROCM, "include")]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    msg = (r.stdout + r.stderr).strip()
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected
    lines = [l for l in msg.splitlines() if "packed-fp32-ops" not in l and "ignoring feature" not in l]
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n" + "\n".join(lines))
    if verbose and lines:
        print("\n".join(lines), flush=True)


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    jobs = []
    for name in sorted(os.listdir(CSRC)):
        src = os.path.join(CSRC, name)
        obj = os.path.join(BUILD, name + ".o")
        if name.endswith(".hip"):
            jobs.append(["hipcc", *HIP_FLAGS, "-c", src, "-o", obj])
        elif name.endswith(".c"):
            jobs.append(["gcc", *C_FLAGS, "-c", src, "-o", obj])
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        for f in [ex.submit(_run, j, verbose) for j in jobs]:
            f.result()
    objs = [j[-1] for j in jobs]
    tmp = LIB + ".tmp"
    # -Bsymbolic: the library's own calls (expert_store_* from moe_ffn_forward,
    # for instance) bind to its own definitions, never to a same-named symbol
    # of the executable (a reference build that still links its CPU
    # src/expert_store.c would otherwise interpose its store on them)
    _run(["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
          f"-L{ROCM}/lib", "-lamdhip64", "-lpthread", f"-Wl,-rpath,{ROCM}/lib", "-Wl,-Bsymbolic"], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
