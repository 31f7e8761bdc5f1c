"""Benchmark of the int4 routed-expert MoE layer on one MI355X.

Headline workload: one Mixtral-8x7B-shape MoE layer decode, M = 1 token:
router GEMV + softmax top-2 on the device, then the fused int4 expert FFN
(gate/up/SiLU, down, weighted combine) over the 2 routed experts; 8 experts
of hidden 4096 / inter 14336, int4 g128, fp16 scales, all resident in HBM.
One step = one MoE layer on one synthetic token (one library call:
wisp_gpu_moe_layer_decode_int4). `value` is the mean device microseconds per
layer over K consecutive layers replayed from one HIP graph (how a serving
loop issues a decode step); the eager, Python-launched figure is reported
beside it (lower is better for both).

Also reported (same JSON line, "extra"): Mixtral M=4 and DeepSeek-V3-shape
decode (256 routed experts + 1 shared, inter 2048, hidden 7168, sigmoid
top-8) for M = 1, 2, 4, each with its dominant-kernel roofline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]
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
EV_ROUTE, EV_PREP, EV_GATEUP, EV_DOWN, EV_COMBINE, EV_PF_GATEUP, EV_PF_DOWN, EV_KINDS = \
    0, 1, 2, 3, 4, 5, 6, 7


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Layer:
    """Device state of one MoE layer workload.

    To measure weights streamed from HBM rather than from the 256 MB
    Infinity Cache, steps rotate over `n_sets` independent expert sets (each
    a full layer of resident experts) and a pool of `n_pool` different input
    tokens (so routing, and with it the touched experts, changes per step).
    """

    def __init__(self, shape, M, seed, n_sets=1, n_pool=16):
        from wisp_amd import moe, synth
        from wisp_amd.hip import DeviceBuffer, Stream, to_device
        self.shape, self.M, self.n_pool = shape, M, n_pool
        rng = np.random.default_rng(seed)
        t0 = time.time()
        keep = range(shape.n_experts) if shape.n_experts <= 8 else ()
        self.arenas = []
        for si in range(n_sets):
            self.arenas.append(moe.ExpertArena(
                shape.n_experts, shape.inter, shape.hidden, shape.group_size,
                lambda e, out, si=si: synth.make_blob(np.random.default_rng([seed, si, e]),
                                                      shape.inter, shape.hidden, shape.group_size,
                                                      expert=e, out=out),
                has_zeros=False, keep_host=keep if si == 0 else ()))
        self.shared_blob = None
        self.shared_dev = None
        if shape.shared:
            self.shared_blob = synth.make_blob(np.random.default_rng([seed, 99999]), shape.inter,
                                               shape.hidden, shape.group_size, expert=99999)
            self.shared_dev = DeviceBuffer(self.shared_blob.nbytes + 16)
            self.shared_dev.upload(self.shared_blob, offset=8)
        log(f"{shape.name} M={M}: {n_sets} expert set(s) resident in {time.time() - t0:.1f}s")
        self.W = synth.make_router(rng, shape.n_experts, shape.hidden)
        self.dW = to_device(self.W)
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
        moe.moe_layer_decode_int4(self.dW.ptr, 0, self.kind, self.logits.ptr, self.idx.ptr,
                                  self.w.ptr, a.table.ptr,
                                  self.shared_dev.ptr + 8 if s.shared else 0, a.layout,
                                  self.xptr(i), self.M, s.top_k, s.n_experts, self.ws,
                                  self.out32.ptr, self.out16.ptr, self.stream.handle)

    def fused_experts(self):
        """True when gate/up and down run in one launch: one token (any
        hidden size; above 32 hidden blocks each gate/up row tile's K axis
        is split over several workgroups); otherwise two launches."""
        return self.M == 1

    def separate_router(self):
        """True when the router GEMV gets its own launch: only for rows longer
        than 8192 (otherwise it runs in router workgroups of the prep launch)."""
        return self.shape.hidden > 8192

    def token_bytes(self):
        """Per pool token: algorithmic HBM bytes (packed + scales; zeros are
        +0 and not read) of the expert kernel (gate, up and down of every
        unique expert), the router and the layer, from the routing the
        device produces for it."""
        from wisp_amd.hip import synchronize
        if self._bytes is None:
            s = self.shape
            mat = (s.inter * s.hidden) // 2 + 2 * (s.inter * s.hidden // s.group_size)
            router = s.n_experts * s.hidden * 2
            out = []
            for t in range(self.n_pool):
                self.step(t)
                synchronize()
                ids = self.idx.download(np.int32, (self.M, s.top_k))
                n_u = len({int(e) for e in ids.reshape(-1)}) + (1 if s.shared else 0)
                out.append({"n_unique": n_u, "experts": 3 * n_u * mat,
                            "router": router, "layer": 3 * n_u * mat + router})
            self._bytes = out
        return self._bytes

    def mean_bytes(self, steps):
        tb = self.token_bytes()
        keys = tb[0].keys()
        return {k: float(np.mean([tb[i % self.n_pool][k] for i in range(steps)])) for k in keys}


def time_layer(layer, steps, warmup):
    """Device time per layer over `steps` consecutive layers, two ways:
    replayed from one HIP graph holding all of them (no host launch cost:
    how a serving loop runs a decode step) and launched eagerly from
    Python; then the per-kernel durations from events around each kernel."""
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
    e0.record(layer.stream.handle)
    graph.launch(layer.stream)
    e1.record(layer.stream.handle)
    synchronize()
    dev_ms = e0.elapsed_ms(e1)
    del graph
    # per-kernel durations: same steps again with events around each kernel
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
    return {"us_per_layer": 1e3 * dev_ms / steps, "eager_us_per_layer": 1e3 * eager_ms / steps,
            "host_us_per_layer": 1e3 * host_ms / steps, "kernel_us": kern}


def cpu_baseline(layer, budget_s=10.0):
    """The oracle's vectorised CPU path (AVX-512 or AVX2, OpenMP over rows)
    on this host: router + top-k + the routed experts' FFN, one token per
    layer, cycling over the same token pool as the GPU steps."""
    from oracle import oracle as O
    s = layer.shape
    blobs = layer.arenas[0].host

    def one(i):
        x = layer.x[i % layer.n_pool, 0].astype(np.float32)
        idx, w, _ = O.router_topk(layer.W.view(np.uint16), None, x, s.top_k, kind=s.router)
        acc = np.zeros(s.hidden, np.float32)
        if layer.shared_blob is not None:
            O.expert_ffn(layer.shared_blob, x, acc, 1.0, fast=True)
        for e, we in zip(idx, w):
            O.expert_ffn(blobs[int(e)], x, acc, float(we), fast=True)
        return acc

    one(0)
    times = []
    t_end = time.perf_counter() + budget_s
    while (time.perf_counter() < t_end and len(times) < 2000) or len(times) < 3:
        t0 = time.perf_counter()
        one(len(times))
        times.append(time.perf_counter() - t0)
    isa = {2: "avx512", 1: "avx2", 0: "scalar"}[O.orc().orc_fast_isa()]
    return {"value": round(1e6 * float(np.median(times)), 1), "unit": "us/layer",
            "cores": int(O.orc().orc_num_threads()), "kind": "port",
            "sample": f"{len(times)} {s.name} M=1 layers (router + top-{s.top_k} experts), median; "
                      f"{isa} OpenMP fp32 path of oracle/wisp_oracle.c",
            "cpu": _cpu_model()}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


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


def measure(layer, steps, warmup):
    r = time_layer(layer, steps, warmup)
    b = layer.mean_bytes(steps)
    us = r["us_per_layer"]
    return {
        "us_per_layer": round(us, 3),
        "eager_us_per_layer": round(r["eager_us_per_layer"], 3),
        "host_us_per_layer": round(r["host_us_per_layer"], 3),
        "layer_hbm_frac": round(b["layer"] / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "n_unique_experts": round(b["n_unique"], 2),
        "kernel_us": {k: round(v, 3) for k, v in r["kernel_us"].items()},
        "experts": {**roofline(b["experts"], r["kernel_us"]["experts"]),
                    "bytes_per_launch": int(b["experts"])},
    }


MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA


def measure_prefill(layer, n_tokens, steps, warmup, seed=2048):
    """DeepSeek-V3-shape prefill grouped GEMM: n_tokens fp16 tokens, top-8
    drawn without replacement from Zipf(1.1) over the 256 routed experts,
    plus the shared expert; timed by HIP events on the launch stream
    (graph replay of `steps` calls, and per-kernel events)."""
    from wisp_amd import _lib, moe, synth
    from wisp_amd.hip import DeviceBuffer, Event, Graph, synchronize, to_device
    s = layer.shape
    rng = np.random.default_rng(seed)
    idx = synth.zipf_topk(rng, n_tokens, s.n_experts, s.top_k)
    w = synth.route_weights(rng, n_tokens, s.top_k)
    x = synth.make_x(rng, n_tokens, s.hidden)
    dx, di, dw = to_device(x), to_device(idx), to_device(w)
    a = layer.arenas[0]
    ws = DeviceBuffer(moe.prefill_workspace_bytes(a.layout, n_tokens, s.top_k, s.n_experts, s.shared))
    out16 = DeviceBuffer(2 * n_tokens * s.hidden)
    st = layer.stream

    def step():
        moe.moe_prefill_int4(a.table.ptr, layer.shared_dev.ptr + 8 if s.shared else 0, a.layout,
                             dx.ptr, n_tokens, di.ptr, dw.ptr, s.top_k, s.n_experts, ws,
                             out16=out16.ptr, stream=st.handle)

    for _ in range(warmup):
        step()
    synchronize()
    graph = Graph(st, lambda: [step() for _ in range(steps)])
    graph.launch(st)
    synchronize()
    e0, e1 = Event(), Event()
    e0.record(st.handle)
    graph.launch(st)
    e1.record(st.handle)
    synchronize()
    ms = e0.elapsed_ms(e1) / steps
    del graph
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
    per_pair = 3 * 2 * s.hidden * s.inter
    flops = per_pair * (pairs_routed + (n_tokens if s.shared else 0))
    tflops = flops / (ms * 1e-3) / 1e12
    gu_flops = 2 * 2 * s.hidden * s.inter * (pairs_routed + (n_tokens if s.shared else 0))
    dn_flops = 2 * s.hidden * s.inter * (pairs_routed + (n_tokens if s.shared else 0))
    used = int((counts > 0).sum()) + (1 if s.shared else 0)
    wbytes = used * synth.expert_bytes_no_zeros(s.inter, s.hidden, s.group_size)
    return {
        "ms_per_layer": round(ms, 4), "tokens": n_tokens,
        "tokens_per_s": round(n_tokens / (ms * 1e-3), 1),
        "flops": flops, "tflops": round(tflops, 2),
        "mfma_frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
        "weight_bytes_unique": wbytes, "weight_hbm_frac": round(wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "group_sizes": {"max": int(counts.max()), "median": float(np.median(counts)),
                        "empty": int((counts == 0).sum())},
        "kernel_ms": {"gate_up": round(gu_ms, 4), "down": round(dn_ms, 4)},
        "gate_up_mfma_frac": round(gu_flops / (gu_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
        "down_mfma_frac": round(dn_flops / (dn_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
    }


def measure_streaming(n_layers=8, steps=256, slot_frac=0.30, seed=55, n_templates=16):
    """Expert-streaming decode: n_layers DeepSeek-V3-shape MoE layers whose
    256 routed experts each live in pinned host RAM, a VRAM LRU of slot_frac
    of all experts (the tier of include/wisp_amd.h section 6), one token per
    step with Zipf(1.1) top-8 routing per layer, the shared expert resident.
    The compute stream is synchronised after every layer, as a real decode
    must (the next layer's routing needs this layer's output). Reports
    us/token over all steps and over the second half (warm), the VRAM hit
    rate (vram_hits / lookups) and the H2D rate, plus the rate of a plain
    run of blob copies for comparison."""
    from wisp_amd import moe, synth, tier
    from wisp_amd.hip import DeviceBuffer, Event, PinnedBuffer, Stream, synchronize, to_device
    s = synth.DSV3
    E, k = s.n_experts, s.top_k
    size = synth.blob_size(s.inter, s.hidden, s.group_size)
    t0 = time.time()
    rng = np.random.default_rng(seed)
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
    xs = to_device(synth.make_x(rng, 16, s.hidden))
    routes = [[synth.zipf_topk(rng, 1, E, k) for _ in range(n_layers)] for _ in range(steps)]
    weights = [[synth.route_weights(rng, 1, k) for _ in range(n_layers)] for _ in range(steps)]
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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline workload only")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the DeepSeek-V3 prefill grouped GEMM (2048 tokens)")
    ap.add_argument("--streaming-only", action="store_true",
                    help="only the 8-layer expert-streaming decode (VRAM tier)")
    ap.add_argument("--stream-steps", type=int, default=256)
    ap.add_argument("--dsv3-decode-only", type=int, default=0, metavar="M",
                    help="only the DeepSeek-V3 decode layer with M tokens (profiling runs)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB 5 times (byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the int4 MoE expert path here is a single-GPU "
              "build; expert-parallel sharding over several GPUs is not run", file=sys.stderr)
        sys.exit(2)

    from wisp_amd import synth
    from wisp_amd.hip import device_count
    if device_count() < 1:
        print("no HIP device visible", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return

    if args.dsv3_decode_only:
        ds = Layer(synth.DSV3, args.dsv3_decode_only, seed=777, n_sets=1)
        r = measure(ds, args.steps, args.warmup)
        print(json.dumps({f"deepseek-v3-decode-m{args.dsv3_decode_only}": r}), flush=True)
        return

    if args.streaming_only:
        r = measure_streaming(steps=args.stream_steps)
        print(json.dumps({"deepseek-v3-streaming-8layers": r}), flush=True)
        return

    if args.prefill_only:
        ds = Layer(synth.DSV3, 1, seed=777, n_sets=1)
        r = measure_prefill(ds, 2048, max(2, min(args.steps, 10)), 2)
        print(json.dumps({"deepseek-v3-prefill-2048": r}), flush=True)
        return

    # 4 Mixtral expert sets (3 GB) so consecutive steps stream cold weights
    head = Layer(synth.MIXTRAL, 1, seed=1234, n_sets=4)
    m = measure(head, args.steps, args.warmup)
    log(f"mixtral M=1: {m['us_per_layer']:.2f} us/layer, kernels {m['kernel_us']}")
    gu = dict(m["experts"])
    gu["traffic"] = load_traffic("mixtral-decode-m1/experts")
    result = {
        "metric": "us per MoE layer, int4 expert decode (Mixtral-8x7B shape, M=1)",
        "value": m["us_per_layer"],
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(m["us_per_layer"] / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "mixtral-8x7b-moe-decode-m1", "hidden": 4096, "inter": 14336,
                   "experts": 8, "top_k": 2, "tokens": 1, "weights": "int4 g128 fp16 scales",
                   "router": "softmax top-2 on device", "expert_sets_rotated": 4,
                   "parallelism": "single-gpu"},
        "layer_hbm_frac": m["layer_hbm_frac"],
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
        head.set_tokens(4, rng)
        extra["mixtral-8x7b-decode-m4"] = measure(head, max(20, args.steps // 2), 5)
        log(f"mixtral M=4: {extra['mixtral-8x7b-decode-m4']}")
        del head
        ds = Layer(synth.DSV3, 1, seed=777, n_sets=1)
        for M in (1, 2, 4):
            if M > 1:
                ds.set_tokens(M, rng)
            key = f"deepseek-v3-decode-m{M}"
            extra[key] = measure(ds, max(20, args.steps // 2), 5)
            log(f"{key}: {extra[key]}")
        extra["deepseek-v3-prefill-2048"] = measure_prefill(ds, 2048, 5, 2)
        log(f"deepseek-v3 prefill: {extra['deepseek-v3-prefill-2048']}")
        del ds
        extra["deepseek-v3-streaming-8layers"] = measure_streaming(steps=args.stream_steps)
        log(f"streaming: {extra['deepseek-v3-streaming-8layers']}")
        result["extra"] = extra
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
