"""GPU parity of the int4 MoE prefill grouped GEMM (wisp_gpu_moe_prefill_int4)
against the CPU oracle's run_moe semantics (shared expert, then routed
experts in rank order, fp32 math), token by token.

Bar: max |gpu - oracle| / max |oracle| <= 1e-2 and cosine >= 0.9999 per token
(tests/gpu_util.py). The prefill keeps h and the per-pair down outputs in
fp16 and dequantises weights to fp16 (as the reference GPU path does), so
it is looser than the decode path but well inside that bar.

Routing shapes cover what the tile list must handle: an expert with more
than one 128-token tile (300 = 128 + 128 + 44), exactly 128, 129, a single
token, experts with no tokens at all, skipped slots (idx = -1), and
Zipf-skewed routing at the DeepSeek-V3 shape."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import assert_close, make_expert
from wisp_amd import moe, synth
from wisp_amd.hip import DeviceBuffer, synchronize, to_device

pytestmark = pytest.mark.gpu


def run_prefill(seed, inter, hidden, gs, n_exp, idx, w, shared, zeros, check_tokens=None,
                accumulate=False):
    T, k = idx.shape
    rng = np.random.default_rng(seed)
    used = sorted({int(e) for e in idx.reshape(-1) if 0 <= e < n_exp})
    arena = moe.ExpertArena(n_exp, inter, hidden, gs,
                            lambda e, out: make_expert(seed, e, inter, hidden, gs, zeros, out),
                            has_zeros=zeros, only=used or [0])
    sh_blob = make_expert(seed, 10_000, inter, hidden, gs, zeros) if shared else None
    sh_dev = None
    if shared:
        sh_dev = DeviceBuffer(sh_blob.nbytes + 16)
        sh_dev.upload(sh_blob, offset=8)
    x = synth.make_x(rng, T, hidden)
    dx = to_device(x)
    di, dw = to_device(idx.astype(np.int32)), to_device(w.astype(np.float32))
    ws = DeviceBuffer(moe.prefill_workspace_bytes(arena.layout, T, k, n_exp, shared))
    out32, out16 = DeviceBuffer(4 * T * hidden), DeviceBuffer(2 * T * hidden)
    base = rng.standard_normal((T, hidden)).astype(np.float32) if accumulate else None
    if accumulate:
        out32.upload(base)
    moe.moe_prefill_int4(arena.table.ptr, sh_dev.ptr + 8 if shared else 0, arena.layout, dx.ptr,
                         T, di.ptr, dw.ptr, k, n_exp, ws, out32.ptr, out16.ptr,
                         accumulate=accumulate)
    synchronize()
    g32 = out32.download(np.float32, (T, hidden))
    g16 = out16.download(np.float16, (T, hidden)).astype(np.float32)
    tokens = range(T) if check_tokens is None else check_tokens
    need = sorted({int(e) for t in tokens for e in idx[t] if 0 <= e < n_exp})
    cache = {e: make_expert(seed, e, inter, hidden, gs, zeros) for e in need}
    dummy = cache[need[0]] if need else sh_blob
    blobs = [cache.get(e, dummy) for e in range(n_exp)]
    for t in tokens:
        want = O.moe_combine(blobs, sh_blob, x[t].astype(np.float32), idx[t], w[t])
        if accumulate:
            want = want + base[t]
        assert_close(g32[t], want, f"token {t} fp32")
        assert_close(g16[t], want, f"token {t} fp16")
    return g32


def skewed_routing(rng, n_exp, k):
    """Per-expert token counts 300, 128, 129, 1, 80 (expert 4: a tile of
    65-96 tokens) and 100 (expert 6: a tile of 97-128), then nothing for
    the rest but a few spread tokens; returns idx [T, k] with distinct
    experts per token."""
    want = {0: 300, 1: 128, 2: 129, 3: 1, 4: 80, 6: 100}
    T = 320
    idx = np.full((T, k), -1, np.int32)
    fill = np.zeros(T, np.int32)
    order = rng.permutation(T)
    # a handful of tokens also use experts 5 and 9; 7, 8 and 10+ stay empty
    for t in order[:7]:
        idx[t, 0] = 5 if t % 2 else 9
        fill[t] = 1
    for e, c in want.items():
        placed = 0
        for t in order:
            if placed == c:
                break
            if fill[t] < k and e not in idx[t]:
                idx[t, fill[t]] = e
                fill[t] += 1
                placed += 1
        assert placed == c
    return idx


@pytest.mark.parametrize("shared,zeros", [(True, False), (False, True), (True, True)])
def test_skewed_groups_and_empty_experts(shared, zeros):
    print(f"prefill skew shared={shared} zeros={zeros}", flush=True)
    rng = np.random.default_rng(5)
    idx = skewed_routing(rng, 16, 4)
    w = synth.route_weights(rng, idx.shape[0], idx.shape[1])
    run_prefill(31, 256, 512, 128, 16, idx, w, shared, zeros)


@pytest.mark.parametrize("gs", [32, 64, 256])
def test_group_sizes(gs):
    print(f"prefill gs={gs}", flush=True)
    rng = np.random.default_rng(gs)
    idx = synth.uniform_topk(rng, 150, 8, 2)
    w = synth.route_weights(rng, 150, 2)
    run_prefill(40 + gs, 256, 512, gs, 8, idx, w, True, gs == 64)


def test_accumulate_no_shared_skipped_slots():
    print("prefill accumulate", flush=True)
    rng = np.random.default_rng(12)
    idx = synth.uniform_topk(rng, 70, 12, 3)
    idx[::5, 1] = -1
    w = synth.route_weights(rng, 70, 3)
    run_prefill(77, 384, 768, 128, 12, idx, w, False, False, accumulate=True)


def test_single_token():
    print("prefill one token", flush=True)
    rng = np.random.default_rng(3)
    idx = synth.uniform_topk(rng, 1, 8, 2)
    w = synth.route_weights(rng, 1, 2)
    run_prefill(3, 256, 512, 128, 8, idx, w, True, False)


def test_dsv3_shape_zipf():
    print("prefill dsv3 zipf 96 tokens", flush=True)
    s = synth.DSV3
    rng = np.random.default_rng(2048)
    T = 96
    idx = synth.zipf_topk(rng, T, s.n_experts, s.top_k)
    w = synth.route_weights(rng, T, s.top_k)
    run_prefill(4096, s.inter, s.hidden, s.group_size, s.n_experts, idx, w, True, False,
                check_tokens=[0, 1, 47, 95])


@pytest.mark.parametrize("gs,zeros", [(64, False), (128, True), (32, False)])
def test_long_k_scales_loaded_per_step(gs, zeros):
    """Hidden 7168 with group size 64, zeros, or group size 32: the gate/up
    scale (and zero) image of a workgroup exceeds the LDS budget, so the
    kernels load scales per K step; the down projection (K = 256) stages
    them in LDS."""
    print(f"prefill long K gs={gs} zeros={zeros}", flush=True)
    rng = np.random.default_rng(700 + gs)
    T, n_exp, k = 48, 8, 2
    idx = synth.zipf_topk(rng, T, n_exp, k)
    w = synth.route_weights(rng, T, k)
    run_prefill(700 + gs, 256, 7168, gs, n_exp, idx, w, True, zeros, check_tokens=[0, 17, 47])


def test_matches_decode_path():
    """Every token of a 64-token prefill against the decode entry point run
    4 tokens at a time (itself checked against the oracle)."""
    print("prefill vs decode", flush=True)
    rng = np.random.default_rng(9)
    inter, hidden, n_exp, k, T, seed = 512, 1024, 32, 4, 64, 91
    idx = synth.zipf_topk(rng, T, n_exp, k)
    w = synth.route_weights(rng, T, k)
    g = run_prefill(seed, inter, hidden, 128, n_exp, idx, w, True, False, check_tokens=[0, 63])
    arena = moe.ExpertArena(n_exp, inter, hidden, 128,
                            lambda e, out: make_expert(seed, e, inter, hidden, 128, False, out),
                            has_zeros=False)
    sh_blob = make_expert(seed, 10_000, inter, hidden, 128, False)
    sh_dev = DeviceBuffer(sh_blob.nbytes + 16)
    sh_dev.upload(sh_blob, offset=8)
    x = synth.make_x(np.random.default_rng(seed), T, hidden)
    ws = DeviceBuffer(moe.decode_workspace_bytes(arena.layout, 4, k, True))
    for t0 in range(0, T, 4):
        dx = to_device(x[t0:t0 + 4])
        di, dw = to_device(idx[t0:t0 + 4].astype(np.int32)), to_device(w[t0:t0 + 4])
        out = DeviceBuffer(4 * 4 * hidden)
        moe.moe_decode_int4(arena.table.ptr, sh_dev.ptr + 8, arena.layout, dx.ptr, 4, di.ptr,
                            dw.ptr, k, n_exp, ws, out32=out.ptr)
        synchronize()
        d = out.download(np.float32, (4, hidden))
        for v in range(4):
            assert_close(g[t0 + v], d[v], f"token {t0 + v} prefill vs decode")


def test_invalid_arguments_are_rejected():
    rng = np.random.default_rng(1)
    blob = synth.make_blob(rng, 256, 512, 128)
    L = moe.layout_from_blob(blob, has_zeros=False)
    ws = DeviceBuffer(moe.prefill_workspace_bytes(L, 4, 2, 8, False))
    d = DeviceBuffer(1 << 16)
    with pytest.raises(Exception):
        moe.moe_prefill_int4(d.ptr, 0, L, d.ptr, 0, d.ptr, d.ptr, 2, 8, ws, d.ptr)
    with pytest.raises(Exception):
        moe.moe_prefill_int4(d.ptr, 0, L, d.ptr, 4, d.ptr, d.ptr, 2, 8, DeviceBuffer(64), d.ptr)
    with pytest.raises(Exception):
        moe.moe_prefill_int4(d.ptr, 0, L, d.ptr + 2, 4, d.ptr, d.ptr, 2, 8, ws, d.ptr)


def test_graph_replays_match_eager():
    """The prefill forks its small tiles onto a second stream and joins it
    back: captured in a HIP graph on the caller's stream (after an eager
    call), every replay gives the eager call's output bit for bit, with
    other eager prefills and synchronisations between the replays. The
    routing has full 128-token tiles (on the caller's stream) and small
    tiles (on the second stream)."""
    from wisp_amd.hip import Graph, Stream
    print("prefill graph replays vs eager", flush=True)
    seed, inter, hidden, gs, n_exp, k = 91, 256, 512, 128, 16, 4
    rng = np.random.default_rng(seed)
    idx = skewed_routing(rng, n_exp, k)
    w = synth.route_weights(rng, idx.shape[0], k)
    T = idx.shape[0]
    arena = moe.ExpertArena(n_exp, inter, hidden, gs,
                            lambda e, out: make_expert(seed, e, inter, hidden, gs, False, out),
                            has_zeros=False)
    sh_blob = make_expert(seed, 10_000, inter, hidden, gs, False)
    sh_dev = DeviceBuffer(sh_blob.nbytes + 16)
    sh_dev.upload(sh_blob, offset=8)
    xs = [to_device(synth.make_x(rng, T, hidden)) for _ in range(2)]
    di, dw = to_device(idx.astype(np.int32)), to_device(w.astype(np.float32))
    ws = [DeviceBuffer(moe.prefill_workspace_bytes(arena.layout, T, k, n_exp, True))
          for _ in range(2)]
    outs = [DeviceBuffer(4 * T * hidden) for _ in range(2)]
    st = Stream()

    def call(i):
        moe.moe_prefill_int4(arena.table.ptr, sh_dev.ptr + 8, arena.layout, xs[i].ptr, T,
                             di.ptr, dw.ptr, k, n_exp, ws[i], outs[i].ptr, stream=st.handle)

    call(0)
    synchronize()
    ref = outs[0].download(np.float32, (T, hidden))
    graph = Graph(st, lambda: call(0))
    for r in range(3):
        outs[0].zero()
        call(1)                       # other eager work on the same stream
        synchronize()
        graph.launch(st)
        synchronize()
        got = outs[0].download(np.float32, (T, hidden))
        assert np.array_equal(got, ref), f"replay {r} differs from the eager call"
    del graph


def test_concurrent_host_threads_match_serial():
    """Two host threads enqueue prefills at the same time, each on its own
    stream with its own workspace and output, while the library's second
    stream (one per device, with shared fork and join events) serves both:
    every output equals the one computed by a single thread, bit for bit."""
    import threading

    from wisp_amd.hip import Stream
    print("prefill from two host threads vs serial", flush=True)
    seed, inter, hidden, gs, n_exp, k = 97, 256, 512, 128, 16, 4
    rng = np.random.default_rng(seed)
    idx = skewed_routing(rng, n_exp, k)
    w = synth.route_weights(rng, idx.shape[0], k)
    T = idx.shape[0]
    arena = moe.ExpertArena(n_exp, inter, hidden, gs,
                            lambda e, out: make_expert(seed, e, inter, hidden, gs, False, out),
                            has_zeros=False)
    sh_blob = make_expert(seed, 20_000, inter, hidden, gs, False)
    sh_dev = DeviceBuffer(sh_blob.nbytes + 16)
    sh_dev.upload(sh_blob, offset=8)
    di, dw = to_device(idx.astype(np.int32)), to_device(w.astype(np.float32))
    n_thr, reps = 2, 6
    xs = [to_device(synth.make_x(rng, T, hidden)) for _ in range(n_thr)]
    ws = [DeviceBuffer(moe.prefill_workspace_bytes(arena.layout, T, k, n_exp, True))
          for _ in range(n_thr)]
    outs = [[DeviceBuffer(4 * T * hidden) for _ in range(reps)] for _ in range(n_thr)]
    streams = [Stream() for _ in range(n_thr)]

    def call(i, r):
        moe.moe_prefill_int4(arena.table.ptr, sh_dev.ptr + 8, arena.layout, xs[i].ptr, T,
                             di.ptr, dw.ptr, k, n_exp, ws[i], outs[i][r].ptr,
                             stream=streams[i].handle)

    ref = []
    for i in range(n_thr):
        call(i, 0)
        streams[i].synchronize()
        ref.append(outs[i][0].download(np.float32, (T, hidden)))
    assert not np.array_equal(ref[0], ref[1])
    errors = []

    def worker(i):
        try:
            for r in range(reps):
                call(i, r)
            streams[i].synchronize()
        except Exception as ex:  # reported below, in the main thread
            errors.append(ex)

    for o in outs:
        for b in o:
            b.zero()
    synchronize()
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(n_thr)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    synchronize()
    for i in range(n_thr):
        for r in range(reps):
            got = outs[i][r].download(np.float32, (T, hidden))
            assert np.array_equal(got, ref[i]), f"thread {i} call {r} differs from the serial call"


def test_many_experts():
    """1,023 routed experts plus the shared one, the most the prefill takes
    (the expert-offset builder keeps a histogram row per wave in LDS): the
    offsets and the tile list cover the top ids, with a 150-token expert
    near the top of the range (a full tile plus a remainder) and the others
    spread over the whole range. One more expert is rejected before any
    launch."""
    print("prefill 1023 experts", flush=True)
    rng = np.random.default_rng(1023)
    n_exp, k, T = 1023, 4, 160
    heavy = 1000
    idx = np.empty((T, k), np.int32)
    for t in range(T):
        others = rng.choice(n_exp - 1, size=k, replace=False)
        others = np.where(others >= heavy, others + 1, others)   # never the heavy expert
        idx[t] = others
        if t < 150:
            idx[t, t % k] = heavy
    idx[0, 1 if idx[0, 0] == heavy else 0] = n_exp - 1
    assert all(len(set(r)) == k for r in idx)
    w = synth.route_weights(rng, T, k)
    run_prefill(77, 256, 512, 128, n_exp, idx, w, True, False,
                check_tokens=[0, 1, 75, 127, 128, 149, 150, T - 1])
    L = moe.layout_from_blob(synth.make_blob(rng, 256, 512, 128), has_zeros=False)
    assert moe.prefill_workspace_bytes(L, T, k, n_exp, True) > 0
    assert moe.prefill_workspace_bytes(L, T, k, n_exp + 1, True) == 0
    d = DeviceBuffer(1 << 16)
    with pytest.raises(Exception):
        moe.moe_prefill_int4(d.ptr, d.ptr, L, d.ptr, 4, d.ptr, d.ptr, 2, n_exp + 1,
                             DeviceBuffer(1 << 20), d.ptr)
