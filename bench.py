"""Benchmark of the int4 routed-expert MoE layer on one MI355X.

Headline workload: one DeepSeek-V3-shape MoE layer decode, M = 1 token:
sigmoid router GEMV + top-8 of 256 routed experts on the device, then the
fused int4 expert FFN (gate/up/SiLU, down, weighted combine) over the 8
routed experts and the always-on shared expert; hidden 7168, inter 2048,
int4 g128, fp16 scales, all resident in HBM. One step = one MoE layer on one
synthetic token (one library call: wisp_gpu_moe_layer_decode_int4).

Cold weights: the 256 MB Infinity Cache could hold a layer's shared expert
and router between steps, so steps rotate over 2 full expert sets (2 x 256
routed experts, 11.6 GB), 16 shared-expert/router variants and a pool of 16
tokens; the same (set, variant, token) recurs only every 16 layers, after
about 3 GB of other weights.

`value` is the median over R >= 5 replays of one HIP graph holding K
consecutive layers (how a serving loop issues decode steps) of the device
microseconds per layer; min and max over the replays are reported beside
it, with the eager (Python-launched) figure. Lower is better.

Also reported ("extra"): DeepSeek-V3 M = 2, 4 and Mixtral-8x7B M = 1, 4
decode layers, the DeepSeek-V3 2048-token prefill grouped GEMM (MFMA
fraction of the routed FLOPs, and with the shared expert), and 8-layer
DeepSeek-V3 expert streaming through the VRAM tier.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--replays R]
                       [--no-cpu] [--quick]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E peak
MFMA_F16_PEAK_TFLOPS = 2500.0   # MI355X dense fp16 MFMA
EV_ROUTE, EV_PREP, EV_GATEUP, EV_DOWN, EV_COMBINE, EV_PF_GATEUP, EV_PF_DOWN, EV_KINDS = \
    0, 1, 2, 3, 4, 5, 6, 7


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Layer:
    """Device state of one MoE decode-layer workload.

    Steps rotate over `n_sets` independent sets of routed experts (each a
    full layer), `n_var` shared-expert + router variants and a pool of
    `n_pool` tokens, so that timed steps read weights from HBM rather than
    from the Infinity Cache.
    """

    def __init__(self, shape, M, seed, n_sets=1, n_var=1, n_pool=16):
        from wisp_amd import moe, synth
        from wisp_amd.hip import DeviceBuffer, Stream, to_device
        self.shape, self.M, self.n_pool, self.seed = shape, M, n_pool, seed
        rng = np.random.default_rng(seed)
        t0 = time.time()
        keep = range(shape.n_experts) if shape.n_experts <= 8 else ()
        self.arenas = []
        for si in range(n_sets):
            self.arenas.append(moe.ExpertArena(
                shape.n_experts, shape.inter, shape.hidden, shape.group_size,
                lambda e, out, si=si: synth.bench_expert(shape, seed, si, e, out),
                has_zeros=False, keep_host=keep if si == 0 else ()))
        self.shared_blobs, self.shared_dev = [], []
        if shape.shared:
            for v in range(n_var):
                b = synth.bench_shared(shape, seed, v)
                d = DeviceBuffer(b.nbytes + 16)
                d.upload(b, offset=8)
                self.shared_blobs.append(b if v == 0 else None)
                self.shared_dev.append(d)
        self.W = [synth.make_router(rng, shape.n_experts, shape.hidden) for _ in range(n_var)]
        self.dW = [to_device(w) for w in self.W]
        self.n_var = n_var
        log(f"{shape.name} M={M}: {n_sets} expert set(s), {n_var} shared/router variant(s) "
            f"resident in {time.time() - t0:.1f}s")
        self.kind = moe.ROUTER_SOFTMAX if shape.router == "softmax" else moe.ROUTER_SIGMOID
        self.stream = Stream()
        self.set_tokens(M, rng)

    def set_tokens(self, M, rng):
        from wisp_amd import moe, synth
        from wisp_amd.hip import DeviceBuffer, to_device
        s = self.shape
        self.M = M
        self.x = synth.make_x(rng, self.n_pool * M, s.hidden).reshape(self.n_pool, M, s.hidden)
        self.dx = to_device(self.x)
        self.logits = DeviceBuffer(4 * M * s.n_experts)
        self.idx = DeviceBuffer(4 * M * s.top_k)
        self.w = DeviceBuffer(4 * M * s.top_k)
        self.ws = DeviceBuffer(moe.decode_workspace_bytes(self.arenas[0].layout, M, s.top_k, s.shared))
        self.out16 = DeviceBuffer(2 * M * s.hidden)
        self.out32 = DeviceBuffer(4 * M * s.hidden)
        self._bytes = None

    def xptr(self, i):
        return self.dx.ptr + (i % self.n_pool) * self.M * self.shape.hidden * 2

    def step(self, i):
        """One MoE layer: router + top-k + experts in one library call."""
        from wisp_amd import moe
        s = self.shape
        a = self.arenas[i % len(self.arenas)]
        v = i % self.n_var
        moe.moe_layer_decode_int4(self.dW[v].ptr, 0, self.kind, self.logits.ptr, self.idx.ptr,
                                  self.w.ptr, a.table.ptr,
                                  self.shared_dev[v].ptr + 8 if s.shared else 0, a.layout,
                                  self.xptr(i), self.M, s.top_k, s.n_experts, self.ws,
                                  self.out32.ptr, self.out16.ptr, self.stream.handle)

    def fused_experts(self):
        """True when gate/up and down run in one launch (one token)."""
        return self.M == 1

    def separate_router(self):
        """True when the router GEMV gets its own launch (rows over 8192)."""
        return self.shape.hidden > 8192

    def token_bytes(self, steps):
        """Per step: algorithmic HBM bytes (packed + scales; zeros are +0 and
        not read) of the expert kernel(s) (gate, up and down of every unique
        expert), the router and the layer, from the routing the device
        produces for that step."""
        from wisp_amd.hip import synchronize
        if self._bytes is None:
            s = self.shape
            mat = (s.inter * s.hidden) // 2 + 2 * (s.inter * s.hidden // s.group_size)
            router = s.n_experts * s.hidden * 2
            period = int(np.lcm.reduce([self.n_pool, len(self.arenas), self.n_var]))
            out = []
            for t in range(period):
                self.step(t)
                synchronize()
                ids = self.idx.download(np.int32, (self.M, s.top_k))
                n_u = len({int(e) for e in ids.reshape(-1)}) + (1 if s.shared else 0)
                out.append({"n_unique": n_u, "experts": 3 * n_u * mat,
                            "router": router, "layer": 3 * n_u * mat + router})
            self._bytes = out
        return [self._bytes[i % len(self._bytes)] for i in range(steps)]

    def mean_bytes(self, steps):
        tb = self.token_bytes(steps)
        return {k: float(np.mean([b[k] for b in tb])) for k in tb[0]}


def time_layer(layer, steps, warmup, replays):
    """Device time per layer over `steps` consecutive layers: replayed from
    one HIP graph holding all of them `replays` times (median, min, max),
    launched eagerly from Python once; then the per-kernel durations from
    events recorded around each kernel on the launch stream."""
    from wisp_amd import _lib
    from wisp_amd.hip import Event, Graph, synchronize
    for i in range(warmup):
        layer.step(i)
    synchronize()
    e0, e1 = Event(), Event()
    t0 = time.perf_counter()
    e0.record(layer.stream.handle)
    for i in range(steps):
        layer.step(i)
    e1.record(layer.stream.handle)
    synchronize()
    host_ms = (time.perf_counter() - t0) * 1e3
    eager_ms = e0.elapsed_ms(e1)
    graph = Graph(layer.stream, lambda: [layer.step(i) for i in range(steps)])
    graph.launch(layer.stream)       # warm replay
    synchronize()
    per = []
    for _ in range(replays):
        e0.record(layer.stream.handle)
        graph.launch(layer.stream)
        e1.record(layer.stream.handle)
        synchronize()
        per.append(1e3 * e0.elapsed_ms(e1) / steps)
    del graph
    evs = [[Event() for _ in range(2 * EV_KINDS)] for _ in range(steps)]
    arrs = [(ctypes.c_void_p * (2 * EV_KINDS))(*[e.handle for e in row]) for row in evs]
    lib = _lib.lib()
    for i in range(steps):
        lib.wisp_amd_set_kernel_events(ctypes.cast(arrs[i], ctypes.c_void_p), EV_KINDS)
        layer.step(i)
    lib.wisp_amd_set_kernel_events(None, 0)
    synchronize()

    def kernel_us(k):
        return 1e3 * float(np.mean([evs[i][2 * k].elapsed_ms(evs[i][2 * k + 1])
                                    for i in range(steps)]))

    kern = {}
    if layer.separate_router():
        kern["router_gemv"] = kernel_us(EV_ROUTE)
    kern["prep"] = kernel_us(EV_PREP)
    if layer.fused_experts():
        kern["experts"] = kernel_us(EV_GATEUP)
    else:
        kern["gate_up"] = kernel_us(EV_GATEUP)
        kern["down"] = kernel_us(EV_DOWN)
        kern["experts"] = kern["gate_up"] + kern["down"]
    return {"us_per_layer": float(np.median(per)), "us_min": float(np.min(per)),
            "us_max": float(np.max(per)), "replays": replays,
            "eager_us_per_layer": 1e3 * eager_ms / steps,
            "host_us_per_layer": 1e3 * host_ms / steps, "kernel_us": kern}


def roofline(nbytes, us):
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def load_traffic(workload):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(workload)
    except (OSError, ValueError):
        return None


def measure(layer, steps, warmup, replays):
    r = time_layer(layer, steps, warmup, replays)
    b = layer.mean_bytes(steps)
    us = r["us_per_layer"]
    return {
        "us_per_layer": round(us, 3),
        "us_min": round(r["us_min"], 3), "us_max": round(r["us_max"], 3),
        "replays": r["replays"], "layers_per_replay": steps,
        "eager_us_per_layer": round(r["eager_us_per_layer"], 3),
        "host_us_per_layer": round(r["host_us_per_layer"], 3),
        "layer_hbm_frac": round(b["layer"] / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "layer_bytes": int(b["layer"]),
        "n_unique_experts": round(b["n_unique"], 2),
        "kernel_us": {k: round(v, 3) for k, v in r["kernel_us"].items()},
        "experts": {**roofline(b["experts"], r["kernel_us"]["experts"]),
                    "bytes_per_launch": int(b["experts"])},
    }


# ---------------------------------------------------------------------------
# CPU baseline (the oracle's C restatement, timed on this host's cores)
# ---------------------------------------------------------------------------

def _cpu_info():
    model, phys, ids = "unknown", set(), {}
    try:
        with open("/proc/cpuinfo") as f:
            pid = core = None
            for ln in f:
                key = ln.split(":", 1)[0].strip()
                if key in ("cpu family", "model", "stepping") and key not in ids:
                    ids[key] = ln.split(":", 1)[1].strip()
                if ln.startswith("model name") and model == "unknown":
                    model = ln.split(":", 1)[1].strip()
                elif ln.startswith("physical id"):
                    pid = ln.split(":", 1)[1].strip()
                elif ln.startswith("core id"):
                    core = ln.split(":", 1)[1].strip()
                    phys.add((pid, core))
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count()
    # family/model/stepping identify the part when the model name is generic
    return {"cpu": model, "cpu_family_model_stepping": "/".join(
                ids.get(k, "?") for k in ("cpu family", "model", "stepping")),
            "logical_cpus_visible": os.cpu_count(), "cpus_in_affinity": aff,
            "physical_cores_visible": len(phys) or None,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def _time_bounded(fn, budget_s, max_runs, min_runs=3):
    fn(0)
    times = []
    t_end = time.perf_counter() + budget_s
    while (time.perf_counter() < t_end and len(times) < max_runs) or len(times) < min_runs:
        t0 = time.perf_counter()
        fn(len(times))
        times.append(time.perf_counter() - t0)
    return times


def cpu_baseline(layer, budget_s=10.0):
    """The oracle's vectorised CPU path (AVX-512 or AVX2, OpenMP over rows)
    on this host for the headline workload: router + top-k + the shared and
    routed experts' FFN, one token per layer, over the same token pool and
    the first expert set and variant of the GPU steps."""
    from oracle import oracle as O
    s = layer.shape
    blobs = layer.arenas[0].host if layer.arenas[0].host else None
    if blobs is None:
        from wisp_amd import synth
        cache = {}

        def blob(e):
            if e not in cache:
                cache[e] = synth.bench_expert(s, layer.seed, 0, e)
            return cache[e]
    else:
        def blob(e):
            return blobs[e]
    shared = layer.shared_blobs[0] if layer.shared_blobs else None

    def one(i):
        x = layer.x[i % layer.n_pool, 0].astype(np.float32)
        idx, w, _ = O.router_topk(layer.W[0].view(np.uint16), None, x, s.top_k, kind=s.router)
        acc = np.zeros(s.hidden, np.float32)
        if shared is not None:
            O.expert_ffn(shared, x, acc, 1.0, fast=True)
        for e, we in zip(idx, w):
            O.expert_ffn(blob(int(e)), x, acc, float(we), fast=True)
        return acc

    for i in range(layer.n_pool):      # make every routed blob of the pool once
        one(i)
    times = _time_bounded(one, budget_s, 5000)
    isa = {2: "avx512", 1: "avx2", 0: "scalar"}[O.orc().orc_fast_isa()]
    return {"value": round(1e6 * float(np.median(times)), 1), "unit": "us/layer",
            "cores": int(O.orc().orc_num_threads()), "kind": "port",
            "sample": f"{len(times)} {s.name} M=1 layers (router + top-{s.top_k} experts"
                      f"{' + shared' if shared is not None else ''}), median; {isa} OpenMP fp32 "
                      f"path of oracle/wisp_oracle.c, about {budget_s:.0f} s of CPU work",
            **_cpu_info()}


def cpu_single_expert(budget_s=8.0):
    """C1: one Mixtral-8x7B-shape expert FFN (x fp16 [1, 4096]) on the CPU:
    the vectorised path and the reference-cost scalar restatement (per-element
    fp16 -> fp32 conversions, as the reference's scalar branch), both OpenMP
    over rows on every thread."""
    from oracle import oracle as O
    from wisp_amd import synth
    s = synth.MIXTRAL
    blob = synth.bench_expert(s, synth.MIXTRAL_BENCH_SEED, 0, 0)
    x = synth.make_x(np.random.default_rng(5), 1, s.hidden)[0].astype(np.float32)
    nbytes = synth.expert_bytes_no_zeros(s.inter, s.hidden, s.group_size)
    out = {}
    for name, fast, budget, runs in (("vectorised", True, budget_s, 2000),
                                     ("scalar_reference_cost", False, budget_s, 10)):
        t = _time_bounded(lambda i: O.expert_ffn(blob, x, None, 1.0, fast=fast), budget, runs)
        us = 1e6 * float(np.median(t))
        out[name] = {"us": round(us, 1), "gbs": round(nbytes / (us * 1e-6) / 1e9, 2),
                     "runs": len(t)}
    isa = {2: "avx512", 1: "avx2", 0: "scalar"}[O.orc().orc_fast_isa()]
    return {"workload": "one mixtral-8x7b expert FFN, int4 g128, 90,832,896 B of weights",
            "threads": int(O.orc().orc_num_threads()), "vectorised_isa": isa, **out}


# ---------------------------------------------------------------------------
# prefill and streaming
# ---------------------------------------------------------------------------

def measure_prefill(layer, n_tokens, steps, warmup, replays):
    """DeepSeek-V3-shape prefill grouped GEMM: n_tokens fp16 tokens, top-8
    drawn without replacement from Zipf(1.1) over the 256 routed experts,
    plus the shared expert (synth.prefill_draw, the draw the config-scale
    parity test checks); timed by HIP events on the launch stream (graph
    replays of `steps` calls, and per-kernel events)."""
    from wisp_amd import _lib, moe, synth
    from wisp_amd.hip import DeviceBuffer, Event, Graph, synchronize, to_device
    s = layer.shape
    idx, w, x = synth.prefill_draw(s, n_tokens)
    dx, di, dw = to_device(x), to_device(idx), to_device(w)
    a = layer.arenas[0]
    ws = DeviceBuffer(moe.prefill_workspace_bytes(a.layout, n_tokens, s.top_k, s.n_experts, s.shared))
    out16 = DeviceBuffer(2 * n_tokens * s.hidden)
    st = layer.stream

    def step():
        moe.moe_prefill_int4(a.table.ptr, layer.shared_dev[0].ptr + 8 if s.shared else 0,
                             a.layout, dx.ptr, n_tokens, di.ptr, dw.ptr, s.top_k, s.n_experts, ws,
                             out16=out16.ptr, stream=st.handle)

    for _ in range(warmup):
        step()
    synchronize()
    graph = Graph(st, lambda: [step() for _ in range(steps)])
    graph.launch(st)
    synchronize()
    e0, e1 = Event(), Event()
    per = []
    for _ in range(replays):
        e0.record(st.handle)
        graph.launch(st)
        e1.record(st.handle)
        synchronize()
        per.append(e0.elapsed_ms(e1) / steps)
    del graph
    ms = float(np.median(per))
    evs = [Event() for _ in range(2 * EV_KINDS)]
    arr = (ctypes.c_void_p * (2 * EV_KINDS))(*[e.handle for e in evs])
    lib = _lib.lib()
    lib.wisp_amd_set_kernel_events(ctypes.cast(arr, ctypes.c_void_p), EV_KINDS)
    step()
    lib.wisp_amd_set_kernel_events(None, 0)
    synchronize()
    gu_ms = evs[2 * EV_PF_GATEUP].elapsed_ms(evs[2 * EV_PF_GATEUP + 1])
    dn_ms = evs[2 * EV_PF_DOWN].elapsed_ms(evs[2 * EV_PF_DOWN + 1])
    counts = np.bincount(idx.reshape(-1), minlength=s.n_experts)
    pairs_routed = int(counts.sum())
    pairs_all = pairs_routed + (n_tokens if s.shared else 0)
    per_pair = 3 * 2 * s.hidden * s.inter
    flops_routed = per_pair * pairs_routed
    flops_all = per_pair * pairs_all
    tf_routed = flops_routed / (ms * 1e-3) / 1e12
    tf_all = flops_all / (ms * 1e-3) / 1e12
    # pairs in the full-tile class (tiles of 65-128 tokens): the kernels that
    # EV_PF_GATEUP / EV_PF_DOWN time, while the smaller tiles run beside
    # them on the library's second stream
    grp = list(counts) + ([n_tokens] if s.shared else [])
    full_pairs = int(sum((c // 128) * 128 + (c % 128 if c % 128 > 64 else 0) for c in grp))
    gu_flops = 2 * 2 * s.hidden * s.inter * full_pairs
    dn_flops = 2 * s.hidden * s.inter * full_pairs
    used = int((counts > 0).sum()) + (1 if s.shared else 0)
    wbytes = used * synth.expert_bytes_no_zeros(s.inter, s.hidden, s.group_size)
    return {
        "ms_per_layer": round(ms, 4), "ms_min": round(float(np.min(per)), 4),
        "ms_max": round(float(np.max(per)), 4), "replays": replays, "tokens": n_tokens,
        "tokens_per_s": round(n_tokens / (ms * 1e-3), 1),
        "flops_routed": flops_routed, "tflops_routed": round(tf_routed, 2),
        "mfma_frac_routed": round(tf_routed / MFMA_F16_PEAK_TFLOPS, 4),
        "flops_with_shared": flops_all, "tflops_with_shared": round(tf_all, 2),
        "mfma_frac_with_shared": round(tf_all / MFMA_F16_PEAK_TFLOPS, 4),
        "weight_bytes_unique": wbytes,
        "weight_hbm_frac": round(wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "group_sizes": {"max": int(counts.max()), "median": float(np.median(counts)),
                        "empty": int((counts == 0).sum())},
        "full_tile_pairs": full_pairs,
        "kernel_ms": {"full_tiles_gate_up": round(gu_ms, 4), "full_tiles_down": round(dn_ms, 4)},
        "full_tiles_gate_up_mfma_frac": round(
            gu_flops / (gu_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
        "full_tiles_down_mfma_frac": round(
            dn_flops / (dn_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
    }


def _header_int(name):
    """An integer #define of include/wisp_amd.h."""
    import re
    hdr = os.path.join(os.path.dirname(os.path.abspath(__file__)), "include", "wisp_amd.h")
    with open(hdr) as f:
        return int(re.search(rf"#define {name} (\d+)", f.read()).group(1))


def measure_block(layer, rows, steps, warmup, replays, per_token_us):
    """The MoE block entry (x += MoE(RMSNorm(x) * w_norm), router on the
    normalised rows) on `rows` drafted tokens of one speculative-verify
    step, on the DeepSeek-V3 layer's rotating expert sets and shared/router
    variants, with a pool of fp32 residual rows updated in place. w_norm is
    scaled by 1e-3: the top-k of the bias-free sigmoid router does not
    depend on the scale of its input, so the routing draws what the plain
    layer call draws, while the MoE adds almost nothing to x, so the rows
    (and their routing) do not drift over the timed calls. Graph replays of
    `steps` calls, HIP events. Beside it, the reference's shape of the same
    work: one single-token layer per drafted token (`per_token_us` each)."""
    from wisp_amd import moe
    from wisp_amd.hip import DeviceBuffer, Event, Graph, synchronize, to_device
    s = layer.shape
    rng = np.random.default_rng(4242 + rows)
    n_pool = 16
    x = rng.standard_normal((n_pool, rows, s.hidden)).astype(np.float32)
    dx = to_device(x)
    norm_w = to_device((1e-3 * (1.0 + 0.05 * rng.standard_normal(s.hidden))).astype(np.float16))
    scores = DeviceBuffer(4 * rows * s.n_experts)
    idx, w = DeviceBuffer(4 * rows * s.top_k), DeviceBuffer(4 * rows * s.top_k)
    ws = DeviceBuffer(moe.block_workspace_bytes(layer.arenas[0].layout, rows, s.top_k,
                                                s.n_experts, s.shared))
    st = layer.stream

    def step(i):
        a = layer.arenas[i % len(layer.arenas)]
        v = i % layer.n_var
        moe.moe_block_int4(dx.ptr + (i % n_pool) * rows * s.hidden * 4, norm_w.ptr, 1e-6,
                           layer.dW[v].ptr, 0, layer.kind, scores.ptr, idx.ptr, w.ptr,
                           a.table.ptr, layer.shared_dev[v].ptr + 8 if s.shared else 0,
                           a.layout, rows, s.top_k, s.n_experts, ws, stream=st.handle)

    def unique_now():
        ids = idx.download(np.int32, (rows, s.top_k))
        return len({int(e) for e in ids.reshape(-1) if e >= 0}) + (1 if s.shared else 0)

    n_unique = []
    for i in range(max(warmup, n_pool)):      # eager calls; the routing each one drew
        step(i)
        synchronize()
        n_unique.append(unique_now())
    graph = Graph(st, lambda: [step(i) for i in range(steps)])
    graph.launch(st)
    synchronize()
    e0, e1 = Event(), Event()
    per = []
    for _ in range(replays):
        e0.record(st.handle)
        graph.launch(st)
        e1.record(st.handle)
        synchronize()
        per.append(1e3 * e0.elapsed_ms(e1) / steps)
    del graph
    n_after = []
    for i in range(n_pool):                   # the same rows after the timed calls
        step(i)
        synchronize()
        n_after.append(unique_now())
    us = float(np.median(per))
    return {"rows": rows, "us_per_call": round(us, 3), "us_min": round(float(np.min(per)), 3),
            "n_unique_experts": round(float(np.mean(n_unique)), 2),
            "n_unique_experts_after": round(float(np.mean(n_after)), 2),
            "us_max": round(float(np.max(per)), 3), "replays": replays,
            "us_per_row": round(us / rows, 3),
            "per_token_loop_us": round(rows * per_token_us, 3),
            "speedup_vs_per_token_loop": round(rows * per_token_us / us, 3),
            "path": "fused decode, calls of up to 4 rows"
                    if rows <= _header_int("WISP_BLOCK_DECODE_MAX_ROWS") else "grouped GEMM"}


def measure_streaming(n_layers=8, steps=256, slot_frac=0.30, seed=55, n_templates=16):
    """Expert-streaming decode: n_layers DeepSeek-V3-shape MoE layers whose
    256 routed experts each live in pinned host RAM, a VRAM LRU of slot_frac
    of all experts (the tier of include/wisp_amd.h section 6), one token per
    step with Zipf(1.1) top-8 routing per layer (synth.streaming_draw), the
    shared expert resident. The compute stream is synchronised after every
    layer, as a real decode must (the next layer's routing needs this
    layer's output). Reports us/token over all steps and over the second
    half (warm), the VRAM hit rate (vram_hits / lookups) and the H2D rate,
    plus the rate of a plain run of blob copies for comparison."""
    from wisp_amd import moe, synth, tier
    from wisp_amd.hip import DeviceBuffer, Event, PinnedBuffer, Stream, synchronize, to_device
    s = synth.DSV3
    E, k = s.n_experts, s.top_k
    size = synth.blob_size(s.inter, s.hidden, s.group_size)
    t0 = time.time()
    temps = [synth.make_blob(np.random.default_rng([seed, i]), s.inter, s.hidden, s.group_size,
                             expert=i) for i in range(n_templates)]
    layers = []
    for l in range(n_layers):
        pb = PinnedBuffer(E * size)
        for e in range(E):
            pb.array[e * size:(e + 1) * size] = temps[(l * E + e) % n_templates]
        layers.append(pb)
    log(f"streaming: {n_layers} x {E} experts ({n_layers * E * size / 1e9:.1f} GB) pinned in "
        f"{time.time() - t0:.1f}s")
    ptrs = [layers[l].ptr + e * size for l in range(n_layers) for e in range(E)]
    layout = moe.layout_from_blob(temps[0], has_zeros=False)
    n_slots = int(round(slot_frac * n_layers * E))
    t = tier.ExpertTier(n_layers, E, size, ptrs, n_slots, scratch_slots=k + 2)
    shared = []
    for l in range(n_layers):
        d = DeviceBuffer(size + 16)
        d.upload(temps[(l + 7) % n_templates], offset=8)
        shared.append(d)
    st = Stream()
    ws = DeviceBuffer(moe.decode_workspace_bytes(layout, 1, k, True))
    out32 = DeviceBuffer(4 * s.hidden)
    xs_h, routes, weights = synth.streaming_draw(s, n_layers, steps, seed=seed)
    xs = to_device(xs_h)
    per_step = []
    half = None
    for step in range(steps):
        if step == steps // 2:
            half = t.stats()
        c0 = time.perf_counter()
        for l in range(n_layers):
            t.moe_decode_layer(l, shared[l].ptr + 8, layout, xs.ptr + (step % 16) * s.hidden * 2, 1,
                               routes[step][l], weights[step][l], ws, out32.ptr, 0, st.handle)
            st.synchronize()
        per_step.append(time.perf_counter() - c0)
    end = t.stats()
    wall = float(np.sum(per_step))
    warm = float(np.sum(per_step[steps // 2:]))
    # plain H2D rate of blob copies, same pinned source, no kernels
    dst = DeviceBuffer(size * 4)
    e0, e1 = Event(), Event()
    from wisp_amd.hip import runtime, check, hipMemcpyHostToDevice
    rt = runtime()
    e0.record(st.handle)
    n_copy = 24
    for i in range(n_copy):
        check(rt.hipMemcpyAsync(dst.ptr + (i % 4) * size, ptrs[(i * 37) % len(ptrs)], size,
                                hipMemcpyHostToDevice, st.handle), "H2D")
    e1.record(st.handle)
    synchronize()
    copy_gbs = n_copy * size / (e0.elapsed_ms(e1) * 1e-3) / 1e9
    wh = {key: end[key] - half[key] for key in end}
    res = {
        "us_per_token": round(1e6 * wall / steps, 1),
        "us_per_token_warm": round(1e6 * warm / (steps - steps // 2), 1),
        "vram_hit_rate": round(end["vram_hits"] / end["lookups"], 4),
        "vram_hit_rate_warm": round(wh["vram_hits"] / wh["lookups"], 4),
        "h2d_gb": round(end["h2d_bytes"] / 1e9, 2),
        "h2d_gbs_during_run": round(end["h2d_bytes"] / wall / 1e9, 2),
        "h2d_gbs_plain_copies": round(copy_gbs, 2),
        "stats": end, "layers": n_layers, "steps": steps, "vram_slots": n_slots,
        "experts_total": n_layers * E, "blob_bytes": size,
    }
    t.close()
    del layers
    return res


def copy_calibration(mib):
    """Five launches of a plain copy of `mib` MiB (source and destination
    both far larger than the Infinity Cache for mib >= 512)."""
    from wisp_amd import _lib
    from wisp_amd.hip import DeviceBuffer, synchronize
    lib = _lib.lib()
    f = lib.wisp_amd__copy_calibration
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    f.restype = ctypes.c_int
    n = mib << 20
    src, dst = DeviceBuffer(n), DeviceBuffer(n)
    src.zero()
    for _ in range(5):
        rc = f(dst.ptr, src.ptr, n, None)
        if rc:
            raise RuntimeError(f"copy calibration failed: hipError {rc}")
    synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "launches": 5}), flush=True)


def dsv3_layer(M):
    from wisp_amd import synth
    return Layer(synth.DSV3, M, seed=synth.DSV3_BENCH_SEED, n_sets=2, n_var=16)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--replays", type=int, default=7)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline workload only")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the DeepSeek-V3 prefill grouped GEMM (2048 tokens)")
    ap.add_argument("--streaming-only", action="store_true",
                    help="only the 8-layer expert-streaming decode (VRAM tier)")
    ap.add_argument("--stream-steps", type=int, default=256)
    ap.add_argument("--dsv3-decode-only", type=int, default=0, metavar="M",
                    help="only the DeepSeek-V3 decode layer with M tokens (profiling runs)")
    ap.add_argument("--mixtral-decode-only", type=int, default=0, metavar="M",
                    help="only the Mixtral-8x7B decode layer with M tokens (profiling runs)")
    ap.add_argument("--verify-only", type=int, default=0, metavar="ROWS",
                    help="only the DeepSeek-V3 MoE block on ROWS drafted tokens (speculative verify)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB 5 times (byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the int4 MoE expert path here is a single-GPU "
              "build; expert-parallel sharding over several GPUs is not run", file=sys.stderr)
        sys.exit(2)
    steps, warmup, replays = max(1, args.steps), max(0, args.warmup), max(5, args.replays)

    from wisp_amd import synth
    from wisp_amd.hip import device_count
    if device_count() < 1:
        print("no HIP device visible", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return

    if args.dsv3_decode_only:
        ds = dsv3_layer(args.dsv3_decode_only)
        r = measure(ds, steps, warmup, replays)
        print(json.dumps({f"deepseek-v3-decode-m{args.dsv3_decode_only}": r}), flush=True)
        return
    if args.mixtral_decode_only:
        mx = Layer(synth.MIXTRAL, args.mixtral_decode_only, seed=synth.MIXTRAL_BENCH_SEED, n_sets=4)
        r = measure(mx, steps, warmup, replays)
        print(json.dumps({f"mixtral-8x7b-decode-m{args.mixtral_decode_only}": r}), flush=True)
        return
    if args.verify_only:
        ds = dsv3_layer(1)
        m1 = measure(ds, steps, warmup, replays)
        r = measure_block(ds, args.verify_only, steps, warmup, replays, m1["us_per_layer"])
        print(json.dumps({f"deepseek-v3-verify-block-{args.verify_only}": r}), flush=True)
        return
    if args.streaming_only:
        r = measure_streaming(steps=args.stream_steps)
        print(json.dumps({"deepseek-v3-streaming-8layers": r}), flush=True)
        return
    if args.prefill_only:
        ds = dsv3_layer(1)
        r = measure_prefill(ds, 2048, max(2, min(steps, 10)), 2, replays)
        print(json.dumps({"deepseek-v3-prefill-2048": r}), flush=True)
        return

    head = dsv3_layer(1)
    m = measure(head, steps, warmup, replays)
    log(f"deepseek-v3 M=1: {m['us_per_layer']:.2f} us/layer (min {m['us_min']:.2f}, "
        f"max {m['us_max']:.2f}), kernels {m['kernel_us']}")
    gu = dict(m["experts"])
    gu["traffic"] = load_traffic("deepseek-v3-decode-m1/experts")
    result = {
        "metric": "us per MoE layer, int4 expert decode (DeepSeek-V3 shape, M=1)",
        "value": m["us_per_layer"],
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(m["us_per_layer"] / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights, fp16 activations, fp32 accumulate",
        "data": "synthetic (seeded int4 weights and fp16 tokens of the named shape)",
        "config": {"workload": "deepseek-v3-moe-decode-m1", "hidden": 7168, "inter": 2048,
                   "routed_experts": 256, "shared_experts": 1, "top_k": 8, "tokens": 1,
                   "weights": "int4 g128 fp16 scales",
                   "router": "sigmoid top-8 on device (uniform-like random choice)",
                   "expert_sets_rotated": 2, "shared_router_variants_rotated": 16,
                   "token_pool": 16, "parallelism": "single-gpu"},
        "us_min": m["us_min"], "us_max": m["us_max"], "replays": m["replays"],
        "layer_hbm_frac": m["layer_hbm_frac"],
        "layer_bytes": m["layer_bytes"],
        "kernel_us": m["kernel_us"],
        "roofline": {"bound": gu["bound"], "achieved": gu["achieved"], "peak": gu["peak"],
                     "unit": gu["unit"], "frac": gu["frac"], "traffic": gu["traffic"],
                     "kernel": "moe experts (int4 gate+up+SiLU and down in one launch)",
                     "bytes_per_launch": gu["bytes_per_launch"]},
    }
    if not args.no_cpu:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(head)
        log(f"cpu baseline {result['cpu_baseline']['value']:.0f} us/layer")

    if not args.quick:
        extra = {}
        rng = np.random.default_rng(99)
        sub = max(16, steps // 2)
        for M in (2, 4):
            head.set_tokens(M, rng)
            key = f"deepseek-v3-decode-m{M}"
            extra[key] = measure(head, sub, 4, replays)
            log(f"{key}: {extra[key]['us_per_layer']} us, kernels {extra[key]['kernel_us']}")
        for rows in (4, 8):
            key = f"deepseek-v3-verify-block-{rows}"
            extra[key] = measure_block(head, rows, sub, 4, replays, m["us_per_layer"])
            log(f"{key}: {extra[key]}")
        extra["deepseek-v3-prefill-2048"] = measure_prefill(head, 2048, 5, 2, replays)
        log(f"deepseek-v3 prefill: {extra['deepseek-v3-prefill-2048']}")
        del head
        mx = Layer(synth.MIXTRAL, 1, seed=synth.MIXTRAL_BENCH_SEED, n_sets=4)
        for M in (1, 4):
            if M > 1:
                mx.set_tokens(M, rng)
            key = f"mixtral-8x7b-decode-m{M}"
            extra[key] = measure(mx, sub, 4, replays)
            log(f"{key}: {extra[key]['us_per_layer']} us, kernels {extra[key]['kernel_us']}")
        del mx
        extra["deepseek-v3-streaming-8layers"] = measure_streaming(steps=args.stream_steps)
        log(f"streaming: {extra['deepseek-v3-streaming-8layers']}")
        if not args.no_cpu:
            extra["cpu_c1_single_mixtral_expert"] = cpu_single_expert()
            log(f"cpu C1: {extra['cpu_c1_single_mixtral_expert']}")
        result["extra"] = extra
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
