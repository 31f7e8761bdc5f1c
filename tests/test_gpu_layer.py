"""GPU parity of the one-call MoE layer decode (wisp_gpu_moe_layer_decode_int4:
router + top-k + shared/routed experts, no host round trip) against the CPU
oracle: routing indices must equal the oracle's wherever the top-k is not
decided by a near-tie of the logits, and the layer output must meet the
fp16 bar of tests/gpu_util.py (max-rel-err <= 1e-2, cosine >= 0.9999).

Also: the result is bit-identical across repeated calls on one workspace
(the down kernel's row-tile counters reset each call and the final sum runs
in a fixed order), and a layer with nothing routed writes zeros."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import assert_close, assert_valid_topk, make_expert
from wisp_amd import moe, synth
from wisp_amd.hip import DeviceBuffer, synchronize, to_device

pytestmark = pytest.mark.gpu


def _keys(W, x, bias, kind):
    """float64 selection keys of one token (a NaN key, never selected, as -inf)."""
    l = W.astype(np.float64) @ x.astype(np.float64)
    b = bias.astype(np.float64) if bias is not None else 0.0
    k = l + b if kind == "softmax" else 1.0 / (1.0 + np.exp(-l)) + b
    return np.where(np.isnan(k), -np.inf, k)


def _scores(W, x, bias, kind):
    """float64 post-activation router scores of one token (softmax over the
    biased logits, or the sigmoid of the raw logits)."""
    l = W.astype(np.float64) @ x.astype(np.float64)
    if kind == "softmax":
        if bias is not None:
            l = l + bias.astype(np.float64)
        z = np.exp(l - np.max(l))
        return z / np.sum(z)
    return 1.0 / (1.0 + np.exp(-l))


def _near_tie(W, x, bias, kind, k):
    """True when two of the k+1 largest selection keys are too close for the
    selection to be decided by fp32 summation order (the logits' fp32 error
    is ~1e-7 here; 2e-5 leaves a wide margin)."""
    key = _keys(W, x, bias, kind)
    srt = np.sort(key[np.isfinite(key)])[::-1]
    return np.min(np.abs(np.diff(srt[: k + 1]))) <= 2e-5 * max(np.max(np.abs(srt)), 1.0)


def run_layer(seed, inter, hidden, n_exp, top_k, M, kind, shared, use_bias, repeat=1,
              gs=128, zeros=False, nan_rows=(), vary_x=False, x32=False):
    """One workspace, `repeat` calls. With vary_x every call routes new tokens
    and each call's output is checked; otherwise the calls repeat one input
    and must agree bit for bit."""
    rng = np.random.default_rng(seed)
    W = synth.make_router(rng, n_exp, hidden, std=0.05)
    for r in nan_rows:
        W[r] = np.float16("nan")
    bias = (rng.standard_normal(n_exp) * 0.1).astype(np.float16) if use_bias else None
    xs = [synth.make_x(rng, M, hidden) for _ in range(repeat if vary_x else 1)]
    # upload only the experts the routing can reach: each token's k + 4 best
    # keys (the slots of the others are never read)
    cand = sorted({int(e) for x in xs for t in range(M)
                   for e in np.argsort(-_keys(W, x[t], bias, kind))[: top_k + 4]})
    arena = moe.ExpertArena(n_exp, inter, hidden, gs,
                            lambda e, out: make_expert(seed, e, inter, hidden, gs, zeros, out),
                            has_zeros=zeros, keep_host=cand, only=cand)
    sh_blob = make_expert(seed, 10_000, inter, hidden, gs, zeros) if shared else None
    sh_dev = None
    if shared:
        sh_dev = DeviceBuffer(sh_blob.nbytes + 16)
        sh_dev.upload(sh_blob, offset=8)
    dW = to_device(W)
    dxs = [to_device(x.astype(np.float32) if x32 else x) for x in xs]
    db = to_device(bias) if use_bias else None
    sc, di, dw = DeviceBuffer(4 * M * n_exp), DeviceBuffer(4 * M * top_k), DeviceBuffer(4 * M * top_k)
    ws = DeviceBuffer(moe.decode_workspace_bytes(arena.layout, M, top_k, shared))
    out32, out16 = DeviceBuffer(4 * M * hidden), DeviceBuffer(2 * M * hidden)
    kcode = moe.ROUTER_SOFTMAX if kind == "softmax" else moe.ROUTER_SIGMOID
    blobs = [arena.host.get(e, arena.host[cand[0]]) for e in range(n_exp)]

    def check(x, g32, g16, gi, gw, gs):
        for t in range(M):
            # the scores output of every expert
            assert np.allclose(gs[t], _scores(W, x[t], bias, kind), rtol=1e-4, atol=1e-7,
                               equal_nan=True), t
            oi, ow, _ = O.router_topk(W.view(np.uint16), bias.view(np.uint16) if use_bias else None,
                                      x[t].astype(np.float32), top_k, kind=kind)
            if _near_tie(W, x[t], bias, kind, top_k):
                # selection decided by rounding: the device's selection must be
                # a top-k of the float64 keys within the tie margin; the
                # experts' math is then checked on that selection
                key = _keys(W, x[t], bias, kind)
                tol = 2e-5 * max(np.max(np.abs(key[np.isfinite(key)])), 1.0)
                assert_valid_topk(key, gi[t], top_k, tol, f"token {t}")
                assert set(gi[t].tolist()) <= set(cand)
                oi, ow = gi[t], gw[t]
            else:
                assert set(oi.tolist()) <= set(cand)
                assert gi[t].tolist() == oi.tolist(), (t, gi[t], oi)
                assert np.allclose(gw[t], ow, rtol=1e-4, atol=1e-6), (t, gw[t], ow)
            assert not set(gi[t].tolist()) & set(nan_rows), (t, gi[t])
            want = O.moe_combine(blobs, sh_blob, x[t].astype(np.float32), oi, ow)
            assert_close(g32[t], want, f"token {t} fp32")
            assert_close(g16[t], want, f"token {t} fp16")

    results = []
    for i in range(repeat):
        xi = i if vary_x else 0
        moe.moe_layer_decode_int4(dW.ptr, db.ptr if use_bias else 0, kcode, sc.ptr, di.ptr, dw.ptr,
                                  arena.table.ptr, sh_dev.ptr + 8 if shared else 0, arena.layout,
                                  dxs[xi].ptr, M, top_k, n_exp, ws, out32.ptr, out16.ptr,
                                  x_dtype=moe.DTYPE_F32 if x32 else moe.DTYPE_F16)
        synchronize()
        g32 = out32.download(np.float32, (M, hidden))
        results.append(g32)
        if vary_x or i == repeat - 1:
            check(xs[xi], g32, out16.download(np.float16, (M, hidden)).astype(np.float32),
                  di.download(np.int32, (M, top_k)), dw.download(np.float32, (M, top_k)),
                  sc.download(np.float32, (M, n_exp)))
    if not vary_x:
        for r in results[:-1]:
            assert np.array_equal(r, results[-1]), "repeated calls differ"
    return results[-1]


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_fused_router_softmax(M):
    print(f"layer softmax fused-router M={M}", flush=True)
    run_layer(500 + M, 256, 512, 8, 2, M, "softmax", shared=(M % 2 == 0), use_bias=(M > 2))


@pytest.mark.parametrize("M", [1, 4])
def test_fused_router_sigmoid_bias(M):
    print(f"layer sigmoid fused-router M={M}", flush=True)
    run_layer(600 + M, 256, 512, 32, 4, M, "sigmoid", shared=True, use_bias=True)


@pytest.mark.parametrize("kind", ["softmax", "sigmoid"])
def test_router_workgroups_in_prep_launch(kind):
    # 256 experts x 1024 hidden x 2 B = 512 KiB router: logits from router
    # workgroups of the prep launch, which the prep workgroup polls
    print(f"layer {kind} router workgroups", flush=True)
    run_layer(700, 256, 1024, 256, 8, 3, kind, shared=True, use_bias=(kind == "sigmoid"))


def test_router_workgroups_consecutive_calls():
    # each call on one workspace must select on its own tokens' logits (the
    # routing words carry a per-call token); 60 experts x 2304 x 2 B =
    # 276 KiB router, so 8 router workgroups, the last with 4 rows
    print("layer router workgroups x4 calls", flush=True)
    run_layer(705, 256, 2304, 60, 4, 4, "softmax", shared=False, use_bias=True, repeat=4,
              vary_x=True)


def test_router_workgroups_fp32_tokens():
    # fp32 activations, 4 tokens, 512 experts: router workgroups of 2 rows
    print("layer router workgroups fp32 x, E=512", flush=True)
    run_layer(707, 256, 1024, 512, 8, 4, "sigmoid", shared=True, use_bias=True, repeat=2,
              vary_x=True, x32=True)


@pytest.mark.parametrize("kind", ["softmax", "sigmoid"])
def test_separate_router_launch(kind):
    # rows of 8320 > 8192: the logits get a launch of their own
    print(f"layer {kind} separate-router", flush=True)
    run_layer(730, 256, 8320, 40, 4, 2, kind, shared=True, use_bias=True, repeat=2, vary_x=True)


def test_one_token_64_experts_router_workgroups():
    # 64 experts x 2304 hidden x 2 B = 288 KiB router: router workgroups,
    # then the one-wave selection at its largest expert count
    print("layer M=1 E=64 router workgroups", flush=True)
    run_layer(710, 256, 2304, 64, 8, 1, "softmax", shared=True, use_bias=True, repeat=3,
              vary_x=True)


@pytest.mark.parametrize("n_exp,k,kind", [(5, 2, "softmax"), (12, 3, "sigmoid"),
                                          (16, 4, "softmax"), (40, 6, "sigmoid")])
def test_one_token_selection_expert_counts(n_exp, k, kind):
    # the one-wave selection ranks against only the LDS keys in use (8, 16,
    # 32 or 64 slots); expert counts inside and at the edge of each bound
    print(f"layer M=1 one-wave selection E={n_exp} k={k} {kind}", flush=True)
    run_layer(740 + n_exp, 256, 512, n_exp, k, 1, kind, shared=(n_exp % 2 == 0),
              use_bias=(kind == "sigmoid"), repeat=2, vary_x=True)


@pytest.mark.parametrize("n_exp,M", [(32, 1), (256, 1), (40, 3), (256, 4)])
def test_sigmoid_nan_logit_never_selected(n_exp, M):
    # a NaN router row gives a NaN key: the oracle's "largest untaken" never
    # picks it, and neither may the device (one-wave selection per token,
    # and the four-wave grouped selection)
    print(f"layer sigmoid NaN row E={n_exp} M={M}", flush=True)
    run_layer(720 + n_exp + M, 256, 512, n_exp, 4, M, "sigmoid", shared=False, use_bias=True,
              nan_rows=(1, 5))


def test_repeated_calls_bit_identical_with_zeros():
    print("layer repeat x3", flush=True)
    run_layer(800, 384, 640, 16, 4, 2, "softmax", shared=True, use_bias=False, repeat=3,
              zeros=True)


@pytest.mark.parametrize("M", [1, 4])
def test_mixtral_layer(M):
    print(f"layer mixtral M={M}", flush=True)
    s = synth.MIXTRAL
    run_layer(900 + M, s.inter, s.hidden, s.n_experts, s.top_k, M, "softmax", shared=False,
              use_bias=False, repeat=2)


def test_dsv3_layer_m1():
    print("layer dsv3 M=1", flush=True)
    s = synth.DSV3
    run_layer(950, s.inter, s.hidden, s.n_experts, s.top_k, 1, "sigmoid", shared=True,
              use_bias=False, repeat=2)


def test_nothing_routed_writes_zeros():
    print("decode nothing routed", flush=True)
    rng = np.random.default_rng(11)
    inter, hidden, n_exp, k, M = 256, 512, 8, 2, 2
    arena = moe.ExpertArena(n_exp, inter, hidden, 128,
                            lambda e, out: make_expert(11, e, inter, hidden, 128, False, out),
                            has_zeros=False, only=[0])
    x = synth.make_x(rng, M, hidden)
    dx = to_device(x)
    di = to_device(np.full((M, k), -1, np.int32))
    dw = to_device(np.full((M, k), 0.5, np.float32))
    ws = DeviceBuffer(moe.decode_workspace_bytes(arena.layout, M, k, False))
    out32, out16 = DeviceBuffer(4 * M * hidden), DeviceBuffer(2 * M * hidden)
    out32.upload(np.full((M, hidden), 7.0, np.float32))
    moe.moe_decode_int4(arena.table.ptr, 0, arena.layout, dx.ptr, M, di.ptr, dw.ptr, k, n_exp, ws,
                        out32.ptr, out16.ptr)
    synchronize()
    assert np.all(out32.download(np.float32, (M, hidden)) == 0.0)
    assert np.all(out16.download(np.float16, (M, hidden)) == 0.0)
    base = np.full((M, hidden), 3.5, np.float32)
    out32.upload(base)
    moe.moe_decode_int4(arena.table.ptr, 0, arena.layout, dx.ptr, M, di.ptr, dw.ptr, k, n_exp, ws,
                        out32.ptr, 0, accumulate=True)
    synchronize()
    assert np.array_equal(out32.download(np.float32, (M, hidden)), base)


@pytest.mark.parametrize("hidden,M", [(7168, 4), (1024, 3)])
def test_decode_graph_replays_match_eager(hidden, M):
    """Captured in a HIP graph on the caller's stream (after an eager
    call), every replay of a 3- or 4-token layer decode gives the eager
    call's routing and output bit for bit, with other eager calls and
    synchronisations between the replays: the per-call counters are reset
    by kernels inside the graph, and the routing epoch carried in the
    workspace advances on every replay. hidden 7168 takes the K-split
    gate/up with its finishing kernel; 1024 the unsplit one."""
    from wisp_amd.hip import Graph, Stream
    print(f"decode graph replays vs eager: hidden={hidden} M={M}", flush=True)
    seed, inter, n_exp, top_k = 53 + M, 256, 32, 8
    rng = np.random.default_rng(seed)
    blobs = [make_expert(seed, e, inter, hidden, 128) for e in range(n_exp)]
    arena = moe.ExpertArena(n_exp, inter, hidden, 128, lambda e, out: blobs[e], has_zeros=False)
    sb = make_expert(seed, 999, inter, hidden, 128)
    sh = DeviceBuffer(sb.nbytes + 16)
    sh.upload(sb, offset=8)
    dW = to_device(synth.make_router(rng, n_exp, hidden, std=0.05))
    xs = [to_device(synth.make_x(rng, M, hidden)) for _ in range(2)]
    bufs = [dict(scores=DeviceBuffer(4 * M * n_exp), idx=DeviceBuffer(4 * M * top_k),
                 w=DeviceBuffer(4 * M * top_k), out=DeviceBuffer(4 * M * hidden),
                 ws=DeviceBuffer(moe.decode_workspace_bytes(arena.layout, M, top_k, True)))
            for _ in range(2)]
    st = Stream()

    def call(i):
        b = bufs[i]
        moe.moe_layer_decode_int4(dW.ptr, 0, moe.ROUTER_SIGMOID, b["scores"].ptr, b["idx"].ptr,
                                  b["w"].ptr, arena.table.ptr, sh.ptr + 8, arena.layout,
                                  xs[i].ptr, M, top_k, n_exp, b["ws"], out32=b["out"].ptr,
                                  stream=st.handle)

    def read(i):
        return (bufs[i]["idx"].download(np.int32, (M, top_k)),
                bufs[i]["out"].download(np.float32, (M, hidden)))

    call(0)
    synchronize()
    ref = read(0)
    assert np.isfinite(ref[1]).all() and np.abs(ref[1]).max() > 0
    graph = Graph(st, lambda: call(0))
    for r in range(3):
        bufs[0]["out"].zero()
        call(1)                       # other eager work on the same stream
        synchronize()
        graph.launch(st)
        synchronize()
        got = read(0)
        assert np.array_equal(got[0], ref[0]), f"replay {r}: routing differs"
        assert np.array_equal(got[1], ref[1]), f"replay {r}: output differs from the eager call"
    del graph
    for b in bufs:
        assert moe.decode_status(b["ws"]) == 0
