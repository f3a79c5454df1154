#!/usr/bin/env python3
"""Throughput of the quantized MoE-FFN layer on one MI355X.

Default workload: a Qwen3-30B-A3B-shaped MoE layer (d=2048, 128 experts,
top-8 renormalised, expert intermediate 768, gate/up Q4_K, down Q6_K, F32
router) at decode batch 1. A step is one moe_ffn_forward call on one token.
Steps rotate over --layers distinct layers (different routers and experts,
all resident in HBM through the ExpertStore) and every step has its own
token, so the routed weights stream from HBM rather than from the 256 MB
last-level cache. The K timed steps are one HIP-graph replay bracketed by
events on the launch stream.

The roofline object prices the whole layer call: its algorithmic bytes
(router, the distinct routed experts' slices, activations) over the measured
time per step, against 8 TB/s; prefill is priced by its expert FLOPs against
the 2.5 PFLOP/s dense bf16 matrix-core peak. `traffic` is the layer's HBM
bytes from FETCH_SIZE / WRITE_SIZE counter runs (profiles/traffic_*.json,
made by --traffic from rocprofv3 output). For the one-token decode plan,
`kernels` prices each of its kernels on its own bytes: each is launched alone
over 8 x layers distinct (layer, token) states and each launch's duration
comes from HIP events that the dispatch itself records
(moe_decode_stage_timed).

cpu_baseline times the reference's own moe_ffn (compiled from its sources
into oracle/_ref) on a bounded sample of the same workload on the host, at 4
OpenMP threads and at every physical core available (OMP_PROC_BIND=close,
median of 10 runs, CPU model stated), or the oracle's restatement where that
library is absent.

The default run then times every other configuration of the benchmark in
the same process - OLMoE Q8_0 at batch 1, OLMoE Q4_K_M at batch 1, 4 and 16,
Qwen3 Q4_K_M at batch 32, the 2048-token Zipf-biased Q8_0 prefill and the
48-layer stack with its LM head - and lists them under `configs`, each with
its time per layer, roofline and CPU baseline (a shorter CPU sample each);
`value` stays the headline's. --only times --workload alone; --phases prints
only the phase breakdown of one-token calls (moe_decode_phases).

Other workloads (--workload) print the same JSON schema: OLMoE shapes,
batched decode and 2048-token prefill.
"""
import argparse
import json
import os
import statistics
import sys
import time

import numpy as np  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
# the CPUs this process may use, read before any OpenMP runtime starts: with
# OMP_PROC_BIND set, loading one (torch does) binds the calling thread to a
# single core, and its affinity then names that core alone
START_CPUS = frozenset(os.sched_getaffinity(0))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer decode tok/s + achieved HBM GB/s (% of peak); prefill tok/s"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 matrix-core peak of one MI355X

WORKLOADS = {
    # name: (shape, tokens per step, layers rotated, router logit bias)
    "qwen3-q4km-decode-b1": ("qwen3-30b-a3b-q4_k_m", 1, 32, False),
    "qwen3-q4km-decode-b32": ("qwen3-30b-a3b-q4_k_m", 32, 8, False),
    "olmoe-q8_0-decode-b1": ("olmoe-q8_0", 1, 24, False),
    "olmoe-q4km-decode-b1": ("olmoe-q4_k_m", 1, 32, False),
    "olmoe-q4km-decode-b4": ("olmoe-q4_k_m", 4, 16, False),
    "olmoe-q4km-decode-b16": ("olmoe-q4_k_m", 16, 8, False),
    "qwen3-q8_0-prefill-2048": ("qwen3-30b-a3b-q8_0", 2048, 2, True),
}
DEFAULT = "qwen3-q4km-decode-b1"
# name: (shape, layers, vocab): greedy decode of a whole MoE stack + Q8_0 LM head
STACKS = {"qwen3-q4km-stack48": ("qwen3-30b-a3b-q4_k_m", 48, 151936)}
# name: (shape, layers, vocab, HBM expert pool bytes): the same stack read from a GGUF file on disk through the
# ExpertStore, its experts paged into a pool smaller than the model
PAGED = {"qwen3-q4km-stack48-paged4g": ("qwen3-30b-a3b-q4_k_m", 48, 151936, 4 << 30)}
# name: (transformer layers, query heads, kv heads, head dim, context tokens, block tokens):
# decode attention over the GPU KV store (dense, every block attended)
ATTN = {"qwen3-attn-ctx4096": (48, 32, 4, 128, 4096, 32)}
# name: (shape, layers, query heads, kv heads, head dim, context tokens, block tokens, vocab): greedy decode of a
# whole model (attention over the KV store + MoE FFN per block, tied Q8_0 head) through vireo_model_step
MODELS = {"qwen3-model-ctx1024": ("qwen3-30b-a3b-q4_k_m", 48, 32, 4, 128, 1024, 32, 151936)}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default: 48 cycles of the layer rotation)")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default=DEFAULT,
                    choices=sorted(WORKLOADS) + sorted(STACKS) + sorted(PAGED) + sorted(ATTN) + sorted(MODELS)
                    + ["copy-512MiB"])
    ap.add_argument("--layers", type=int, default=None, help="distinct layers rotated through")
    ap.add_argument("--tokens", type=int, default=None,
                    help="tokens per layer call of --workload (default: the workload's own)")
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--traffic", nargs=4, metavar=("FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE"),
                    help="no GPU run: read four rocprofv3 --pmc output directories (FETCH_SIZE and WRITE_SIZE of "
                         "this workload, then of --workload copy-512MiB) and write profiles/traffic_<workload>.json")
    ap.add_argument("--only", action="store_true",
                    help="time only --workload (the default run also times every other configuration)")
    ap.add_argument("--phases", action="store_true",
                    help="only the per-phase breakdown of one-token calls (moe_decode_phases), no timed replay")
    ap.add_argument("--plan", type=int, default=0,
                    help="execution plan (vireo_hip_set_path): 0 automatic, 1 decode, 2 grouped, 3 fused, 4 fp32")
    return ap.parse_args()


def alg_bytes_layer(shape, idx, B):
    """Router + distinct routed experts' slices + activations (x in/out, hb)."""
    distinct = len(np.unique(idx.reshape(-1)))
    return shape.E * shape.d * 4 + distinct * shape.expert_bytes() + 3 * B * shape.d * 4, distinct


def alg_bytes_stages(shape):
    """Algorithmic bytes of each kernel of the one-token decode plan, each
    charged with the weights it computes on:
      route   the F32 router, hb, the router parts written;
      gate/up the k routed experts' gate and up slices, hb, the parts, the
              expert table, the k x fe activations written (the down rows it
              touches ahead of the down kernel are charged to the down kernel);
      down    the k experts' down slices, the activations, x read and written."""
    gs, us, ds = shape.slice_bytes()
    E, d, k, fe = shape.E, shape.d, shape.k, shape.fe
    return {"route": E * d * 4 + d * 4 + E * 16,
            "topk_gateup": k * (gs + us) + d * 4 + E * 16 + E * 3 * 8 + k * fe * 4,
            "down_combine": k * ds + k * fe * 4 + 2 * d * 4}


def expert_flops(shape, B):
    """FLOPs of the expert projections of a call: gate, up and down, 2 d fe
    each per (token, routed expert)."""
    return 6 * B * shape.k * shape.d * shape.fe


def layer_traffic(workload):
    """HBM bytes per layer call measured with rocprofv3 counters
    (profiles/traffic_<workload>.json, written by --traffic), or None."""
    tf = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    if not os.path.exists(tf):
        return None, None
    with open(tf) as f:
        t = json.load(f)
    return t.get("hbm_bytes_per_layer"), t


def host_cpu():
    """The host's CPU model and the physical cores this process may use: the
    cores of the CPUs in its affinity mask, capped by OMP_NUM_THREADS where
    the environment sets it (a GPU machine's share of a larger host)."""
    model, cores, cur, smt = "unknown", {}, {}, 1
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "processor":
                    cur = {"cpu": int(v)}
                elif k == "model name":
                    model = v
                elif k in ("physical id", "core id", "siblings", "cpu cores"):
                    cur[k] = v
                if "cpu" in cur and "physical id" in cur and "core id" in cur:
                    cores[cur["cpu"]] = (cur["physical id"], cur["core id"])
                if "siblings" in cur and "cpu cores" in cur and int(cur["cpu cores"]) > 0:
                    smt = max(1, int(cur["siblings"]) // int(cur["cpu cores"]))
    except (OSError, ValueError):
        pass
    allowed = START_CPUS
    phys = len({cores[c] for c in allowed if c in cores})
    # a virtualised /proc/cpuinfo may give every CPU the same core id: then
    # count the CPUs available divided by the hardware threads per core
    phys = max(phys, len(allowed) // smt)
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return model, phys, min(phys, cap) if cap > 0 else phys


def _omp_threads(n):
    """Set the thread count of the OpenMP runtime the reference library uses
    (the system libgomp, which it links)."""
    import ctypes
    ctypes.CDLL("libgomp.so.1").omp_set_num_threads(int(n))


def _timed_runs(run, per_run, runs, first):
    """runs timings of per_run consecutive tokens each (tokens first,
    first + 1, ...): microseconds per token of every run."""
    out, t = [], first
    for _ in range(runs):
        t0 = time.perf_counter()
        for _ in range(per_run):
            run(t)
            t += 1
        out.append((time.perf_counter() - t0) / per_run * 1e6)
    return out, t


def cpu_baseline(shape, B, seed, seconds):
    """The reference's moe_ffn on the host: tokens one at a time, as the
    reference runs them (it has no batched path), weights warm in RAM, with
    OMP_PROC_BIND=close; timed at 4 OpenMP threads (the reference's default,
    src/gguf_run.c:267) and at every physical core available, the median of
    10 runs each. The all-core figure is the value."""
    from vireo_amd import workloads as W
    model, phys, all_cores = host_cpu()
    g, u, d = W.host_layer(shape, 0, seed)
    router = W.host_router(shape, 0, seed)
    warm, n_tok = 24, 4096
    x, hb = W.host_hidden(shape.d, n_tok, seed, stream=W.stream_id(0, W.KIND_HIDDEN) + 7)
    from oracle.oracle import Reference, RefMoE, Oracle
    if Reference.available():
        rm = RefMoE(Reference(), shape, [router], [g], [u], [d])
        run = lambda t: rm.run(0, x[t % n_tok:t % n_tok + 1], hb[t % n_tok:t % n_tok + 1])  # noqa: E731
        kind = "reference"
    else:
        o = Oracle()
        gs, us, ds = shape.slice_bytes()
        G = [g[e * gs:(e + 1) * gs] for e in range(shape.E)]
        U = [u[e * us:(e + 1) * us] for e in range(shape.E)]
        D = [d[e * ds:(e + 1) * ds] for e in range(shape.E)]
        run = lambda t: o.moe_ffn(shape, router, G, U, D, x[t % n_tok:t % n_tok + 1],  # noqa: E731
                                  hb[t % n_tok:t % n_tok + 1])
        rm = None
        kind = "port"
    runs, res, t = 10, {}, 0
    for threads in dict.fromkeys((4, all_cores)):
        if kind == "reference":
            _omp_threads(threads)
        for _ in range(warm):  # page every expert the sample will touch into RAM, start the threads
            run(t)
            t += 1
        t0 = time.perf_counter()
        run(t)
        t += 1
        one = time.perf_counter() - t0
        # 10 runs within about seconds / 2 per thread count
        per_run = max(3, min(200, int(seconds / 2 / runs / max(one, 1e-6))))
        us, t = _timed_runs(run, per_run, runs, t)
        res[threads] = (statistics.median(us), per_run, us)
    if rm is not None:
        rm.close()
    us_all, per_run, _ = res[all_cores]
    us_4 = res[4][0]
    return {"value": round(1e6 / us_all, 3), "unit": "tok/s", "cores": all_cores, "kind": kind,
            "cpu_model": model, "physical_cores_available": phys, "omp_proc_bind": os.environ.get("OMP_PROC_BIND"),
            "statistic": f"median of {runs} runs of {per_run} tokens",
            "sample": f"single-token {shape.name} MoE-layer calls through the reference's moe_ffn (one layer, "
                      f"weights warm in RAM), {runs} runs per thread count, OMP_PROC_BIND=close, "
                      f"{all_cores} threads = every physical core available ({model})",
            "us_per_layer": round(us_all, 1),
            "threads_4": {"value": round(1e6 / us_4, 3), "unit": "tok/s", "us_per_layer": round(us_4, 1),
                          "note": "4 OpenMP threads, the reference's default (src/gguf_run.c:267)"}}


def cpu_baseline_stack(shape, L, vocab, seed, seconds):
    """Host time per token of the stack: L x the reference's moe_ffn on one
    layer (cpu_baseline) plus its gguf_matmul of the Q8_0 LM head, timed on
    a slice of the head's rows and scaled to the vocabulary (the matmul is
    row-parallel)."""
    from vireo_amd import workloads as W
    from oracle.oracle import Reference, Oracle
    layer = cpu_baseline(shape, 1, seed, seconds)
    rows = 16384
    head = W.host_matrix(W.Q8_0, shape.d, 0, rows, seed, W.stream_id(0, W.KIND_LM_HEAD))
    x = W.host_normal(shape.d, seed, 99)
    lib = Reference() if Reference.available() else Oracle()
    if layer["kind"] == "reference":
        _omp_threads(layer["cores"])
    lib.matmul(W.Q8_0, head, x, shape.d, rows)
    times = []
    for _ in range(10):
        t0 = time.perf_counter()
        lib.matmul(W.Q8_0, head, x, shape.d, rows)
        times.append(time.perf_counter() - t0)
    head_s = statistics.median(times) * vocab / rows
    tok_s = 1.0 / (L * layer["us_per_layer"] * 1e-6 + head_s)
    out = dict(layer)
    out.update({"value": round(tok_s, 4),
                "sample": f"{layer['sample']}; times {L} layers, plus the LM head matmul timed on {rows} of its "
                          f"{vocab} rows (median of 10, {head_s * 1e3:.1f} ms scaled)",
                "lm_head_ms": round(head_s * 1e3, 2)})
    out["threads_4"] = dict(layer["threads_4"], value=None,
                            note="per-layer figure only (the 4-thread head matmul is not timed)")
    return out


def bench_stack(args):
    print(json.dumps(stack_result(args, args.workload, args.cpu_seconds)), flush=True)


def stack_result(args, workload, cpu_seconds, steps=None):
    """Greedy decode through moe_stack_step: embedding row (the tied LM head),
    RMSNorm + MoE layer x L, RMSNorm, Q8_0 LM head, argmax; K steps captured
    in one HIP graph, each step reading the token the previous one wrote."""
    import torch
    from vireo_amd import _lib
    from vireo_amd import stack as S
    from vireo_amd import workloads as W

    lib = _lib.load()
    _lib.check(lib.vireo_hip_init(0), "vireo_hip_init")
    _lib.check(lib.vireo_hip_set_path(args.plan), "vireo_hip_set_path")
    shape_name, L, vocab = STACKS[workload]
    L = args.layers or L
    shape = W.SHAPES[shape_name]
    K = steps or args.steps or 128
    Wm = args.warmup if args.warmup is not None else 2
    print(f"[bench] {workload}: building {L} layers of {shape.name} and a [{vocab} x {shape.d}] Q8_0 LM head",
          file=sys.stderr, flush=True)
    st = S.DeviceStack(shape, L, vocab=vocab, seed=args.seed)
    token = torch.full((1,), 17, dtype=torch.int32, device="cuda")
    for _ in range(max(1, Wm)):  # the first step pins every layer's leases
        st.step(token)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(K):
            st.step(token, stream=s)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    ms_per_step = ms / K
    # algorithmic bytes of one token: per layer the router, the k selected
    # experts and the activations; the LM head; the embedding row
    layer_b = shape.E * shape.d * 4 + shape.k * shape.expert_bytes() + 2 * shape.d * 4
    tok_b = L * layer_b + vocab * W.row_bytes(W.Q8_0, shape.d) + W.row_bytes(W.Q8_0, shape.d) + vocab * 4
    gbs = tok_b / (ms_per_step / 1e3) / 1e9
    result = {
        "metric": METRIC, "value": round(K / (ms / 1e3), 2), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": Wm,
        "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{L}-layer {shape.name} MoE stack (attention omitted) + Q8_0 LM head "
                               f"[{vocab} x {shape.d}], greedy decode batch 1",
                   "layers": L, "d": shape.d, "experts": shape.E, "top_k": shape.k, "ffn_exp": shape.fe,
                   "vocab": vocab, "tied_embedding": True},
        "us_per_layer": round(ms_per_step * 1e3 / L, 3),
        "token_alg_bytes": int(tok_b), "step_GBps": round(gbs, 1),
        "roofline": {"kernel": "moe_stack_step (all kernels of a step)", "bound": "hbm", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
    }
    st.close()
    del st, g
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    if not args.no_cpu:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline_stack(shape, L, vocab, args.seed, cpu_seconds)
    return result


def bench_paged_stack(args):
    """The stack of bench_stack served from a GGUF file through an
    ExpertStore whose HBM pool holds a fraction of the experts: every layer's
    routed experts not resident are read from the file (the page cache) into
    the pool on the copy stream before their kernels run, and the experts the
    next layer's router guesses are read while each layer's routing is on its
    way. Steps are timed one by one (a paged step makes host decisions between
    layers, so it is not captured in a graph); the pool's counters give the
    bytes paged per token, read-ahead included."""
    import tempfile
    import torch
    from vireo_amd import _lib
    from vireo_amd import gguf as G
    from vireo_amd import workloads as W

    lib = _lib.load()
    _lib.check(lib.vireo_hip_init(0), "vireo_hip_init")
    shape_name, L, vocab, cap = PAGED[args.workload]
    L = args.layers or L
    shape = W.SHAPES[shape_name]
    K = args.steps or 8
    Wm = args.warmup if args.warmup is not None else 2
    tmp = tempfile.mkdtemp(prefix="vireo_paged_")
    path = os.path.join(tmp, "stack.gguf")
    try:
        print(f"[bench] {args.workload}: writing {L} layers of {shape.name} ({L * shape.E * shape.expert_bytes() / 2**30:.1f} "
              f"GiB of experts) and a [{vocab} x {shape.d}] Q8_0 head to {path}", file=sys.stderr, flush=True)
        # the experts are made on the device (the host generator's bytes) and copied out layer by layer
        from vireo_amd import moe as M
        dm = M.DeviceMoE(shape, L, seed=args.seed)
        G.write_moe_gguf(path, shape, L, seed=args.seed, vocab=vocab,
                         progress=lambda msg: print(f"[bench] {msg}", file=sys.stderr, flush=True),
                         layer_bytes=dm.device_layer_bytes)
        dm.close()
        del dm
        torch.cuda.empty_cache()
        print(f"[bench] loading with a {cap / 2**30:.1f} GiB expert pool", file=sys.stderr, flush=True)
        m = G.GGUFModel(path, expert_capacity=cap)
        d = shape.d
        x = torch.empty(d, dtype=torch.float32, device="cuda")
        xb = torch.empty_like(x)
        logits = torch.empty(vocab, dtype=torch.float32, device="cuda")
        token = torch.full((1,), 17, dtype=torch.int32, device="cuda")
        stream = torch.cuda.Stream()  # a stream of its own, as a serving loop would pass
        for i in range(Wm):
            m.step(token, x, xb, logits, stream=stream)
            torch.cuda.synchronize()
            print(f"[bench] warm-up step {i} done", file=sys.stderr, flush=True)
        before, pf0 = m.hbm_stats(), m.prefetch_stats()
        t0 = time.perf_counter()
        for i in range(K):
            m.step(token, x, xb, logits, stream=stream)
            torch.cuda.synchronize()
            print(f"[bench] step {i} done", file=sys.stderr, flush=True)
        secs = time.perf_counter() - t0
        after, pf1 = m.hbm_stats(), m.prefetch_stats()
        paged = after["bytes_read"] - before["bytes_read"]
        misses = after["misses"] - before["misses"]
        ms_per_step = secs * 1e3 / K
        gbs = paged / K / (ms_per_step / 1e3) / 1e9
        result = {
            "metric": METRIC, "value": round(K / secs, 3), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": Wm,
            "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f32", "data": "synthetic",
            "config": {"workload": f"{L}-layer {shape.name} MoE stack (attention omitted) + Q8_0 LM head "
                                   f"[{vocab} x {shape.d}] from a GGUF file, experts paged into a "
                                   f"{cap / 2**30:.1f} GiB HBM pool, greedy decode batch 1",
                       "layers": L, "experts": shape.E, "top_k": shape.k, "pool_bytes": cap,
                       "model_expert_bytes": L * shape.E * shape.expert_bytes()},
            "paged_bytes_per_token": int(paged / K), "pool_misses_per_token": round(misses / K, 2),
            "prefetch_per_token": {"read_ahead": round((pf1["issued"] - pf0["issued"]) / K, 2),
                                   "used": round((pf1["used"] - pf0["used"]) / K, 2),
                                   "bytes": int((pf1["bytes"] - pf0["bytes"]) / K)},
            "pool": after,
            "roofline": {"kernel": "moe_stack_step with paging (file -> pinned staging -> HBM pool)", "bound": "pcie",
                         "achieved": round(gbs, 2), "unit": "GB/s", "traffic": None,
                         "note": "paged bytes per second of decode; the page-ins cross PCIe from the page cache"},
        }
        m.close()
    finally:
        try:
            os.remove(path)
        except OSError:
            pass
        os.rmdir(tmp)
    print(json.dumps(result), flush=True)


def copy_calibration(args):
    """A plain device-to-device copy of 512 MiB, the reference kernel whose
    HBM counters (FETCH_SIZE, WRITE_SIZE) calibrate the traffic of the MoE
    kernels, and a measure of the bandwidth a streaming kernel reaches."""
    import torch
    n = 512 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    reps = args.steps or 20
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    gbs = 2 * n / (ms / 1e3) / 1e9
    print(json.dumps({"metric": "device copy GB/s (read + write)", "value": round(gbs, 1), "unit": "GB/s",
                      "n_gpus": 1, "steps": reps, "warmup": 3, "ms_per_step": round(ms, 4),
                      "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
                      "data": "synthetic", "config": {"workload": "copy 512 MiB", "bytes_read": n, "bytes_written": n},
                      "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}), flush=True)


def cpu_baseline_attn(L, H, KVH, hd, ctx, G, seed, seconds):
    """The reference's dense KV store (src/kvstore_dense.c, from oracle/_ref)
    attending one layer's query heads at the same context on the host,
    scaled to the whole model's layers."""
    from oracle.oracle import Reference, RefKV
    if not Reference.available():
        return None
    ref = Reference()
    rng = np.random.default_rng(seed)
    kv = RefKV(ref, KVH, hd, G)
    for t in range(ctx):
        k = rng.standard_normal((KVH, hd)).astype(np.float32)
        v = rng.standard_normal((KVH, hd)).astype(np.float32)
        for h in range(KVH):
            kv.append(h, t, k[h], v[h])
    q = rng.standard_normal((H, hd)).astype(np.float32)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for h in range(H):
            kv.attend(h // (H // KVH), q[h])
        n += 1
    dt = time.perf_counter() - t0
    kv.close()
    us_layer = dt / n * 1e6
    return {"value": round(1e6 / (us_layer * L), 3), "unit": "tok/s", "cores": 1, "kind": "reference",
            "sample": f"{n} layers of {H}-head attention at context {ctx} through the reference's dense store "
                      f"(one host thread), {dt:.1f} s, scaled to {L} layers",
            "us_per_layer": round(us_layer, 1)}


def bench_attn(args):
    """Decode attention of a Qwen3-30B-A3B-shaped model over the GPU KV store:
    a step appends one token's keys and values to every layer's kv heads and
    attends its query heads over the whole context. The store is contiguous
    and the position lives on the device (vireo_kv_append_pos /
    vireo_kv_attend_gqa_pos), so the K timed steps are one HIP-graph replay.
    Algorithmic bytes per step are the keys and values of the context, read
    once per kv head."""
    import torch
    from vireo_amd import _lib
    from vireo_amd import kv as KV
    _lib.check(_lib.load().vireo_hip_init(0), "vireo_hip_init")
    L, H, KVH, hd, ctx, G = ATTN[args.workload]
    K = args.steps or 64
    Wm = args.warmup if args.warmup is not None else 2
    dev = torch.device("cuda:0")
    print(f"[bench] {args.workload}: filling {ctx} tokens of {L} x {KVH} kv heads", file=sys.stderr, flush=True)
    kv = KV.DeviceKV(L * KVH, hd, G, dense=True, max_tokens=ctx + K)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    kbuf = torch.randn((64, KVH, hd), generator=gen, device=dev)
    vbuf = torch.randn((64, KVH, hd), generator=gen, device=dev)
    s = torch.cuda.current_stream()
    p0 = ctx - K // 2  # the timed steps cover positions p0 .. p0 + K - 1 (mean context ctx)
    for t in range(p0):  # the context before the measured steps
        for l in range(L):
            kv.append(l * KVH, t, kbuf[(t + l) % 64], vbuf[(t + 7 * l) % 64], stream=s)
    q = torch.randn((H, hd), generator=gen, device=dev)
    out = torch.empty((H, hd), device=dev)
    pos = torch.full((1,), p0, dtype=torch.int32, device=dev)
    one = torch.ones(1, dtype=torch.int32, device=dev)

    def step(st):
        for l in range(L):
            kv.append_pos(l * KVH, pos, kbuf[l % 64], vbuf[(7 * l) % 64], stream=st)
            kv.attend_gqa_pos(l * KVH, H, KVH, pos, q, out, stream=st)
        pos.add_(one)
    for _ in range(Wm):  # uncaptured: the first attention call sizes the store's buffers
        step(s)
    torch.cuda.synchronize()
    gs = torch.cuda.Stream()
    gs.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=gs):
        for _ in range(K):
            step(gs)
    torch.cuda.synchronize()
    pos.fill_(p0)
    graph.replay()  # untimed: the same positions as the timed replay
    torch.cuda.synchronize()
    pos.fill_(p0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    assert int(pos.item()) == p0 + K
    ms = e0.elapsed_time(e1)
    ms_step = ms / K
    kv_bytes = L * KVH * ctx * hd * 2 * 4  # the mean context of the timed steps
    gbs = kv_bytes / (ms_step / 1e3) / 1e9
    result = {
        "metric": "decode attention tok/s over the GPU KV store (context 4096)", "value": round(K / (ms / 1e3), 2),
        "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": Wm, "ms_per_step": round(ms_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{L}-layer attention, {H} query heads over {KVH} kv heads of {hd}, context {ctx}, "
                               f"blocks of {G} tokens, contiguous dense store, steps in one HIP graph",
                   "layers": L, "heads": H, "kv_heads": KVH, "head_dim": hd, "context": ctx, "block_tokens": G},
        "us_per_layer": round(ms_step * 1e3 / L, 3), "kv_bytes_per_step": kv_bytes,
        "roofline": {"kernel": "every kernel of a step (append, attention, merge)", "bound": "hbm",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
    }
    kv.close()
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_attn(L, H, KVH, hd, ctx, G, args.seed, args.cpu_seconds)
    print(json.dumps(result))


def cpu_baseline_model(shape, L, H, KVH, hd, ctx, G, vocab, attn_types, seed, seconds):
    """Host time per token of the whole model: the MoE stack's (cpu_baseline_stack)
    plus, per block, the reference's gguf_matmul of the four attention matrices
    and its dense KV store attending every query head at the context, each timed
    on one block and scaled to L blocks."""
    from vireo_amd import workloads as W
    from oracle.oracle import Reference, RefKV
    if not Reference.available():
        return None
    ref = Reference()
    stack = cpu_baseline_stack(shape, L, vocab, seed, seconds)
    d, nq, nk = shape.d, H * hd, KVH * hd
    mats = [(t, n, r, W.host_matrix(t, n, 0, r, seed, 200 + i))
            for i, (t, (n, r)) in enumerate(zip(attn_types, [(d, nq), (d, nk), (d, nk), (nq, d)]))]
    xs = {n: W.host_normal(n, seed, 99) for n in (d, nq)}
    n, t0 = 0, time.perf_counter()
    while n < 3 or time.perf_counter() - t0 < 1.0:
        for t, cols, rows, w in mats:
            ref.matmul(t, w, xs[cols], cols, rows)
        n += 1
    mat_s = (time.perf_counter() - t0) / n
    rng = np.random.default_rng(seed)
    kv = RefKV(ref, KVH, hd, G)
    for t in range(ctx):
        for h in range(KVH):
            kv.append(h, t, rng.standard_normal(hd).astype(np.float32), rng.standard_normal(hd).astype(np.float32))
    q = rng.standard_normal((H, hd)).astype(np.float32)
    n, t0 = 0, time.perf_counter()
    while n < 2 or time.perf_counter() - t0 < 1.0:
        for h in range(H):
            kv.attend(h // (H // KVH), q[h])
        n += 1
    att_s = (time.perf_counter() - t0) / n
    kv.close()
    tok_s = 1.0 / (1.0 / stack["value"] + L * (mat_s + att_s))
    return {"value": round(tok_s, 4), "unit": "tok/s", "cores": stack["cores"], "kind": "reference",
            "sample": f"{stack['sample']}; plus per block the attention matmuls ({mat_s * 1e3:.2f} ms) and "
                      f"{H}-head attention at context {ctx} through the dense store ({att_s * 1e3:.2f} ms, one "
                      f"thread), each timed on one block and scaled to {L}"}


def bench_model(args):
    """Greedy decode of a whole Qwen3-30B-A3B-shaped model through
    vireo_model_step_pos: per block RMSNorm, q/k/v matvecs, per-head QK-norm,
    RoPE, KV append, grouped-query attention over the context, output matvec,
    then the MoE FFN; final norm, Q8_0 LM head (tied embedding), argmax. The
    contiguous KV store is first filled to the context with synthetic keys and
    values; the position and the token live on the device, so the K timed
    steps are one HIP-graph replay (each step reads the token and position
    the previous one wrote)."""
    import torch
    from vireo_amd import _lib
    from vireo_amd import model as MD
    from vireo_amd import workloads as W
    lib = _lib.load()
    _lib.check(lib.vireo_hip_init(0), "vireo_hip_init")
    shape_name, L, H, KVH, hd, ctx, G, vocab = MODELS[args.workload]
    L = args.layers or L
    shape = W.SHAPES[shape_name]
    K = args.steps or 32
    Wm = args.warmup if args.warmup is not None else 2
    attn_types = (W.Q4_K, W.Q4_K, W.Q6_K, W.Q4_K)
    print(f"[bench] {args.workload}: building {L} blocks (attention {H}/{KVH} x {hd} + {shape.name} MoE) and "
          f"the LM head; filling {ctx - Wm} tokens of context", file=sys.stderr, flush=True)
    m = MD.DeviceModel(shape, L, H, KVH, hd, vocab=vocab, max_pos=ctx + K + 8, seed=args.seed,
                       attn_types=attn_types, block_tokens=G, contiguous=True)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    kbuf = torch.randn((64, KVH, hd), generator=gen, device=dev)
    vbuf = torch.randn((64, KVH, hd), generator=gen, device=dev)
    s = torch.cuda.current_stream()
    p0 = ctx - Wm
    for t in range(p0):
        for l in range(L):
            m.kv.append(l * KVH, t, kbuf[(t + l) % 64], vbuf[(t + 7 * l) % 64], stream=s)
    m.pos.fill_(p0)
    for _ in range(Wm):  # uncaptured: first calls pin expert leases and size buffers
        m.step_pos()
    torch.cuda.synchronize()
    tok0 = int(m.token.item())
    gs = torch.cuda.Stream()
    gs.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=gs):
        for _ in range(K):
            m.step_pos(stream=gs)
    torch.cuda.synchronize()

    def replay():
        m.pos.fill_(ctx)
        m.token.fill_(tok0)
        graph.replay()
    replay()  # untimed: the same positions and tokens as the timed replay
    torch.cuda.synchronize()
    m.pos.fill_(ctx)
    m.token.fill_(tok0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    assert int(m.pos.item()) == ctx + K
    ms = e0.elapsed_time(e1)
    ms_step = ms / K
    # algorithmic bytes of one token: per block the attention matrices, the
    # keys and values of the context, and the MoE layer (router, k experts,
    # activations); the LM head and the embedding row
    layer_b = (m.attn_bytes + KVH * (ctx + K // 2) * hd * 2 * 4 + shape.E * shape.d * 4 +
               shape.k * shape.expert_bytes() + 2 * shape.d * 4)
    tok_b = L * layer_b + vocab * W.row_bytes(W.Q8_0, shape.d) + W.row_bytes(W.Q8_0, shape.d) + vocab * 4
    gbs = tok_b / (ms_step / 1e3) / 1e9
    result = {
        "metric": "whole-model decode tok/s (attention over the KV store + MoE FFN, batch 1)",
        "value": round(K / (ms / 1e3), 2), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": Wm,
        "ms_per_step": round(ms_step, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{L}-block {shape.name}-shaped model: attention {H} query / {KVH} kv heads of {hd} "
                               f"(wq, wk Q4_K, wv Q6_K, wo Q4_K), context {ctx}, MoE FFN, Q8_0 LM head "
                               f"[{vocab} x {shape.d}] tied, greedy decode batch 1, steps in one HIP graph",
                   "layers": L, "heads": H, "kv_heads": KVH, "head_dim": hd, "context": ctx, "block_tokens": G,
                   "vocab": vocab},
        "us_per_layer": round(ms_step * 1e3 / L, 3), "token_alg_bytes": int(tok_b),
        "roofline": {"kernel": "vireo_model_step (all kernels of a step)", "bound": "hbm", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
    }
    m.close()
    if not args.no_cpu:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline_model(shape, L, H, KVH, hd, ctx, G, vocab, attn_types, args.seed,
                                                    args.cpu_seconds)
    print(json.dumps(result), flush=True)


# The kernels one layer call launches, by workload (name prefixes as the
# kernel trace reports them), for the per-layer traffic.
LAYER_KERNELS = {
    "decode": ("route_parts_kernel", "decode_gateup_kernel", "down_combine_kernel"),
}


def kernel_short_name(name):
    """A kernel's bare name out of a profiler's demangled signature:
    "void (anonymous namespace)::foo_kernel<8, 1>(int, ...)" -> "foo_kernel"."""
    n = name.replace("(anonymous namespace)::", "").strip()
    if n.startswith("void "):
        n = n[5:]
    return n.split("(")[0].split("<")[0].split("::")[-1].strip()


def _counter_medians(d, counter):
    """Median per dispatch of `counter` (KiB) for every kernel name in the
    rocprofv3 CSV files under directory d."""
    import csv
    import glob
    vals = {}
    for fn in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        with open(fn) as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                name = row["Kernel_Name"]
                vals.setdefault(name, {}).setdefault(row.get("Dispatch_Id", len(vals)), 0.0)
                vals[name][row.get("Dispatch_Id")] += float(row["Counter_Value"])
    return {k: (float(np.median(list(v.values()))), len(v)) for k, v in vals.items()}


def traffic_report(args):
    """HBM traffic per layer call from counter runs: FETCH_SIZE and WRITE_SIZE
    (KiB per dispatch, the median over the run) of each kernel the layer
    launches, each scaled by what the same counter reads for a plain copy of
    512 MiB (whose bytes are known), summed over the layer's kernels."""
    fetch, write, cfetch, cwrite = (_counter_medians(d, c) for d, c in zip(
        args.traffic, ("FETCH_SIZE", "WRITE_SIZE", "FETCH_SIZE", "WRITE_SIZE")))
    copy_kib = 512 * 1024
    cf = max(cfetch.values(), key=lambda v: v[0])[0]
    cw = max(cwrite.values(), key=lambda v: v[0])[0]
    f_factor, w_factor = copy_kib / cf, copy_kib / cw
    prefixes = LAYER_KERNELS["decode"]
    per_kernel, total = {}, 0.0
    for name in sorted(fetch):
        short = kernel_short_name(name)
        if not any(short.startswith(p) for p in prefixes):
            continue
        fk, n = fetch[name]
        wk = write.get(name, (0.0, 0))[0]
        b = fk * 1024 * f_factor + wk * 1024 * w_factor
        per_kernel[name] = {"fetch_kib_median": round(fk, 1), "write_kib_median": round(wk, 1), "dispatches": n,
                            "hbm_bytes": int(b)}
        total += b
    run = f"python3 <repo>/bench.py --workload {args.workload} --no-cpu --steps 96"
    copy = "python3 <repo>/bench.py --workload copy-512MiB --steps 3"
    out = {"workload": args.workload, "hbm_bytes_per_layer": int(total), "kernels": per_kernel,
           "calibration": {"copy_kib": copy_kib, "fetch_kib": round(cf, 1), "write_kib": round(cw, 1),
                           "fetch_factor": round(f_factor, 4), "write_factor": round(w_factor, 4)},
           "commands": [f"cd /tmp && export TMPDIR=/tmp && timeout -s KILL 120 rocprofv3 --pmc {c} --output-format csv "
                        f"-d <out>/{d} -o run -- {cmd}"
                        for c, d, cmd in (("FETCH_SIZE", "fetch", run), ("WRITE_SIZE", "write", run),
                                          ("FETCH_SIZE", "copy_fetch", copy), ("WRITE_SIZE", "copy_write", copy))]
                       + [f"python3 <repo>/bench.py --workload {args.workload} --traffic <out>/fetch <out>/write "
                          "<out>/copy_fetch <out>/copy_write"]}
    path = os.path.join(ROOT, "profiles", f"traffic_{args.workload}.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))


def main():
    args = parse()
    if args.traffic:
        return traffic_report(args)
    if args.workload == "copy-512MiB":
        return copy_calibration(args)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the MoE path here is built and timed on a single MI355X "
              f"(no collectives, no sharding); --gpus {args.gpus} / WORLD_SIZE {world} is not supported.",
              file=sys.stderr)
        sys.exit(2)
    if args.workload in PAGED:
        # no OpenMP binding here: once torch loads the OpenMP runtime it would
        # bind this thread to one core, and the ExpertStore's reader threads,
        # started from it, would inherit that single core
        return bench_paged_stack(args)
    # The CPU baseline binds its OpenMP threads to neighbouring cores, as the
    # reference's baseline plan asks; the runtime reads this when it starts
    # (nothing has loaded it yet: torch is imported below).
    os.environ.setdefault("OMP_PROC_BIND", "close")
    if args.workload in STACKS:
        return bench_stack(args)
    if args.workload in ATTN:
        return bench_attn(args)
    if args.workload in MODELS:
        return bench_model(args)
    if args.phases:
        return layer_result(args, args.workload, args.cpu_seconds)
    result = layer_result(args, args.workload, args.cpu_seconds)
    if args.workload == DEFAULT and not args.only:
        # every other configuration of the layer benchmark, timed in this run
        # with a shorter CPU sample each (the headline `value` stays the
        # default workload's)
        sub = args.cpu_seconds / 2
        result["configs"] = [compact(layer_result(args, w, sub)) for w in ALL_CONFIGS]
        result["configs"].append(compact(stack_result(args, STACK_CONFIG, sub, steps=128)))
    print(json.dumps(result), flush=True)


# the other benchmark configurations the default run times after the headline
ALL_CONFIGS = ["olmoe-q8_0-decode-b1", "olmoe-q4km-decode-b1", "olmoe-q4km-decode-b4", "olmoe-q4km-decode-b16",
               "qwen3-q4km-decode-b32", "qwen3-q8_0-prefill-2048"]
STACK_CONFIG = "qwen3-q4km-stack48"


def compact(r):
    """One configuration's entry of the default run's `configs` list."""
    out = {"workload": r["config"]["workload"], "tok_s": r["value"], "ms_per_step": r["ms_per_step"],
           "steps": r["steps"], "us_per_layer": r.get("us_per_layer"), "config": r["config"],
           "roofline": r.get("roofline"), "cpu_baseline": r.get("cpu_baseline")}
    for key in ("layer_alg_bytes", "distinct_experts", "layer_GBps", "token_alg_bytes", "step_GBps"):
        if key in r:
            out[key] = r[key]
    return out


def layer_result(args, workload, cpu_seconds):
    """One MoE-layer workload (WORKLOADS): its timed HIP-graph replay, the
    roofline, for one-token calls the per-kernel prices and the phase
    breakdown, and the CPU baseline; returns the JSON object (prints only the
    --phases form)."""
    import torch
    from vireo_amd import _lib
    from vireo_amd import moe as M
    from vireo_amd import workloads as W

    lib = _lib.load()
    _lib.check(lib.vireo_hip_init(0), "vireo_hip_init")
    _lib.check(lib.vireo_hip_set_path(args.plan), "vireo_hip_set_path")
    dev = torch.device("cuda:0")
    shape_name, B, L, biased = WORKLOADS[workload]
    headline = workload == args.workload
    L = (args.layers if headline else None) or L
    B = (args.tokens if headline else None) or B
    shape = W.SHAPES[shape_name]
    K = (args.steps if headline else None) or (48 * L if B < 64 else 8 * L)
    Wm = args.warmup if args.warmup is not None else L
    bias = W.zipf_bias(shape.E, 1.1, seed=args.seed) if biased else None
    print(f"[bench] {workload}: building {L} layers of {shape.name} on the GPU", file=sys.stderr, flush=True)
    m = M.DeviceMoE(shape, L, seed=args.seed, logit_bias=bias)

    # a distinct token per step for decode, and at least the 8 x layers tokens
    # that the per-stage timing of the decode plan launches over
    n_tok = max(K, 8 * L) if B == 1 else min(K, 4 * L) * B
    x0, hb0 = W.host_hidden(shape.d, min(n_tok, 4096), args.seed, stream=W.stream_id(0, W.KIND_HIDDEN) + 1)
    reps = (n_tok + x0.shape[0] - 1) // x0.shape[0]
    hb_all = torch.from_numpy(np.tile(hb0, (reps, 1))[:n_tok]).to(dev)
    x_all = torch.from_numpy(np.tile(x0, (reps, 1))[:n_tok]).to(dev)
    steps_tok = n_tok // B

    def step(i, x=x_all, hb=hb_all):
        j = i % steps_tok
        m.forward(i % L, x[j * B:(j + 1) * B], hb[j * B:(j + 1) * B])

    for l in range(L):  # pin every layer and size the workspace outside the timed graph
        step(l)
    if args.phases:
        if B != 1:
            raise SystemExit("--phases: one-token workloads only")
        if args.plan not in (0, 1, 5):
            raise SystemExit("--phases: plans 0, 1 (three decode kernels) and 5 (one layer kernel) carry the stamps")
        print(json.dumps({"workload": workload, "plan": args.plan,
                          "phases": decode_phases(m, shape, L, x_all, hb_all, dev, args.plan)}), flush=True)
        m.close()
        return None
    for i in range(Wm):
        step(i)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(K):
            step(i)
    torch.cuda.synchronize()
    g.replay()  # untimed replay: first-launch costs of the graph
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    ms_per_step = ms / K
    value = K * B / (ms / 1e3)

    # routing of one pass, for the algorithmic byte count
    idx, _ = m.forward(0, x_all[:B].clone(), hb_all[:B], return_routing=True)
    lb, distinct = alg_bytes_layer(shape, idx.cpu().numpy(), B)
    layer_gbs = lb / (ms_per_step / 1e3) / 1e9

    result = {
        "metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": Wm,
        "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{shape.name} MoE layer, {'prefill' if B > 64 else 'decode'} batch {B}",
                   "d": shape.d, "experts": shape.E, "top_k": shape.k, "ffn_exp": shape.fe,
                   "renorm": shape.renorm, "types": [W.TYPE_NAMES[t] for t in (shape.gate_type, shape.up_type,
                                                                                shape.down_type)],
                   "tokens_per_step": B, "layers_rotated": L, "plan": args.plan, "router_bias": "log Zipf(1.1)" if biased else None},
        "us_per_layer": round(ms_per_step * 1e3, 3),
        "layer_alg_bytes": int(lb), "distinct_experts": int(distinct),
        "layer_GBps": round(layer_gbs, 1), "layer_frac_hbm_peak": round(layer_gbs / HBM_PEAK_GBS, 4),
    }

    traffic, _ = layer_traffic(workload) if args.plan == 0 else (None, None)
    if B >= 64:  # prefill: the expert GEMMs run on the matrix cores
        tflops = expert_flops(shape, B) / (ms_per_step / 1e3) / 1e12
        result["roofline"] = {"kernel": "moe_ffn_forward (every kernel of the layer call)", "bound": "mfma",
                              "achieved": round(tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                              "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": traffic,
                              "flops_per_step": expert_flops(shape, B),
                              "hbm": {"achieved": round(layer_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                      "frac": round(layer_gbs / HBM_PEAK_GBS, 4), "alg_bytes": int(lb)}}
    else:
        result["roofline"] = {"kernel": "moe_ffn_forward (every kernel of the layer call)", "bound": "hbm",
                              "achieved": round(layer_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(layer_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                              "alg_bytes_per_launch": int(lb)}
    if B == 1 and lib.moe_decode_state_bytes(M.C.byref(m.model)) > 0:
        result["roofline"]["kernels"] = decode_stage_roofline(m, shape, L, x_all, hb_all, dev)
        if headline:
            result["phases"] = decode_phases(m, shape, L, x_all, hb_all, dev, args.plan)
    m.close()
    del m, g, x_all, hb_all
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    if not args.no_cpu:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(shape, B, args.seed, cpu_seconds)
    return result


# Phases of the one-token decode kernels as moe_decode_phases records them
# (per kernel, the stamp slots after slot 0 = the workgroup's start), for the
# three-kernel plan and for the one-launch layer kernel.
PHASES_3K = {0: ["router part"], 1: ["router parts loaded", "top-k chosen", "first gate/up row", "gate/up rows done"],
             2: ["down plan loaded", "first down row", "down rows done", "combine written"]}
PHASES_1K = {0: ["router part", "parts received", "top-k chosen", "first gate/up row", "activations published",
                 "activations received", "down + combine written"]}
PHASES_SLOTS = {0: ["router part published", "parts received", "top-k chosen", "first gate/up row",
                    "slot's activations received", "down rows computed", "combine written"]}
STAMP_HZ = 100e6  # s_memrealtime


def phase_breakdown(stamps, one_launch_names=None):
    """The critical path of one-token layer calls from moe_decode_phases
    stamps [n x 3*256*8]: per kernel, its first workgroup's start, the spread
    of its workgroups' starts, and for each phase the time at which the last
    workgroup reached it; the gap between one kernel's last phase and the next
    kernel's first start is the kernel boundary. Returns the median over calls
    of each step in microseconds, in order, and the share of calls whose top-k
    took the exact-logit path."""
    st = stamps.reshape(stamps.shape[0], 3, 256, 8).astype(np.int64)
    present = [kk for kk in range(3) if (st[:, kk, :, 0] > 0).any()]
    if not present:  # a build whose kernels carry no stamps
        return [], None
    names = PHASES_3K if len(present) == 3 else (one_launch_names or PHASES_SLOTS)
    steps, exact = {}, []
    for call in st:
        prev_end, t0 = None, None
        for kk in present:
            wg = call[kk][call[kk][:, 0] > 0]
            start = wg[:, 0].min()
            t0 = start if t0 is None else t0
            if prev_end is not None:
                steps.setdefault(f"k{kk} boundary (previous kernel's last phase -> first workgroup start)",
                                 []).append(start - prev_end)
            steps.setdefault(f"k{kk} workgroup start spread", []).append(wg[:, 0].max() - start)
            last = start
            for i, nm in enumerate(names[kk], start=1):
                t = wg[:, i].max()
                steps.setdefault(f"k{kk} {nm}", []).append(t - last)
                last = t
            prev_end = last
        steps.setdefault("total (first start -> last phase)", []).append(prev_end - t0)
        if len(present) == 3:
            exact.append(bool((call[1][:, 7] == 1).any()))
    out = [{"step": k, "us": round(float(np.median(v)) / STAMP_HZ * 1e6, 3)} for k, v in steps.items()]
    return out, (round(float(np.mean(exact)), 4) if exact else None)


def decode_phases(m, shape, L, x_all, hb_all, dev, plan=0):
    """moe_decode_phases over 8 x layers distinct (layer, token) calls captured
    in one HIP graph (replayed twice, the second replay read back)."""
    import torch
    n = 8 * L
    layers = [j % L for j in range(n)]
    x = x_all[:n].clone()
    hb = hb_all[:n].contiguous()
    stamps = torch.zeros((n, 3 * 256 * 8), dtype=torch.int64, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        m.decode_phases(layers, x, hb, stream=s, stamps=stamps)
    torch.cuda.synchronize()
    g.replay()
    g.replay()
    torch.cuda.synchronize()
    steps, exact = phase_breakdown(stamps.cpu().numpy(), PHASES_1K if plan == 5 else None)
    return {"calls": n, "source": "moe_decode_phases (s_memrealtime per workgroup and phase, one HIP graph)",
            "steps": steps, "exact_path_share": exact}


def decode_stage_roofline(m, shape, L, x_all, hb_all, dev):
    """Each kernel of the one-token decode plan alone over NS distinct
    (layer, token) states: moe_decode_stage_timed launches a stage back to
    back and reads every launch's begin and end from HIP events recorded by
    the dispatch itself (hipExtLaunchKernelGGL), the timestamps a kernel
    trace reports. Each kernel is priced against HBM on its own bytes."""
    import torch
    NS = 8 * L
    if x_all.shape[0] < NS or hb_all.shape[0] < NS:
        raise ValueError(f"stage timing needs {NS} token rows, have {x_all.shape[0]}")
    states = m.decode_states(NS)
    idx = torch.empty((NS, shape.k), dtype=torch.int32, device=dev)
    w = torch.empty((NS, shape.k), dtype=torch.float32, device=dev)
    x = x_all[:NS].clone()
    hb = hb_all[:NS]
    layers = [j % L for j in range(NS)]
    names = {0: ("route", "route_parts_kernel (router logits and bounds)"),
             1: ("topk_gateup", "decode_gateup_kernel (top-k, gate/up SwiGLU, down rows touched ahead)"),
             2: ("down_combine", "down_combine_kernel (down projections, weighted combine, residual)")}
    alg = alg_bytes_stages(shape)
    out = []
    for stage in (0, 1, 2):
        us = m.decode_stage_timed(stage, layers, x, hb, states, idx, w)
        key, kname = names[stage]
        avg = float(us.mean())
        if avg <= 0.0:  # the fused plan: stage 1 did the down work too
            continue
        gbs = alg[key] / (avg * 1e-6) / 1e9
        out.append({"stage": key, "kernel": kname, "avg_launch_us": round(avg, 3),
                    "median_launch_us": round(float(np.median(us)), 3), "launches": NS,
                    "alg_bytes_per_launch": alg[key], "achieved": round(gbs, 1), "unit": "GB/s",
                    "frac": round(gbs / HBM_PEAK_GBS, 4)})
    return out


if __name__ == "__main__":
    main()
