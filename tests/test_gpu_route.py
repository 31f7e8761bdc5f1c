"""GPU parity of routing: top-k selection (bit-exact incl. ties), the
router, the expert-offset builder, gather and the weighted combine."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import assert_valid_topk
from wisp_amd import moe, synth
from wisp_amd.hip import DeviceBuffer, synchronize, to_device

pytestmark = pytest.mark.gpu


def brute_topk(keys, k):
    order = sorted(range(len(keys)), key=lambda e: (-keys[e], e))
    return order[:k]


@pytest.mark.parametrize("n_exp,k,ties", [(8, 2, False), (256, 8, True), (256, 8, False), (1024, 64, True)])
def test_topk_from_logits_softmax_bit_exact(n_exp, k, ties):
    print(f"topk n_exp={n_exp} k={k} ties={ties}", flush=True)
    rng = np.random.default_rng(n_exp + k)
    T = 16
    if ties:
        logits = (rng.integers(0, 7, (T, n_exp)) / 3.0).astype(np.float32)
    else:
        logits = rng.standard_normal((T, n_exp)).astype(np.float32) * 3
    dl = to_device(logits)
    sc, di, dw = DeviceBuffer(4 * T * n_exp), DeviceBuffer(4 * T * k), DeviceBuffer(4 * T * k)
    moe.topk_from_logits(dl.ptr, 0, T, n_exp, k, moe.ROUTER_SOFTMAX, sc.ptr, di.ptr, dw.ptr)
    synchronize()
    idx = di.download(np.int32, (T, k))
    w = dw.download(np.float32, (T, k))
    for t in range(T):
        assert idx[t].tolist() == brute_topk(logits[t], k)
        l = logits[t].astype(np.float64)
        p = np.exp(l[idx[t]] - l.max())
        assert np.allclose(w[t], p / p.sum(), rtol=1e-5)
        # selection on logits == oracle selection on the probabilities
        p_all = np.exp(l - l.max()); p_all /= p_all.sum()
        if not ties:
            oi, _ = O.topk_select(p_all.astype(np.float32), k)
            assert idx[t].tolist() == oi.tolist()


def test_topk_sigmoid_with_bias():
    rng = np.random.default_rng(5)
    T, n_exp, k = 8, 256, 8
    logits = rng.standard_normal((T, n_exp)).astype(np.float32) * 2
    bias = (rng.standard_normal(n_exp) * 0.2).astype(np.float16)
    dl, db = to_device(logits), to_device(bias)
    sc, di, dw = DeviceBuffer(4 * T * n_exp), DeviceBuffer(4 * T * k), DeviceBuffer(4 * T * k)
    moe.topk_from_logits(dl.ptr, db.ptr, T, n_exp, k, moe.ROUTER_SIGMOID, sc.ptr, di.ptr, dw.ptr)
    synchronize()
    idx = di.download(np.int32, (T, k))
    w = dw.download(np.float32, (T, k))
    for t in range(T):
        s = 1 / (1 + np.exp(-logits[t].astype(np.float64)))
        key = s + bias.astype(np.float64)
        want = brute_topk(key, k)
        srt = np.sort(key)[::-1]
        gap = np.min(np.abs(np.diff(srt[: k + 1])))
        if gap > 1e-5:
            assert idx[t].tolist() == want
        assert np.allclose(w[t], s[idx[t]] / s[idx[t]].sum(), rtol=1e-5)


@pytest.mark.parametrize("shape,T", [(synth.MIXTRAL, 4), (synth.DSV3, 4), (synth.DSV3, 1)])
def test_router_vs_oracle(shape, T):
    print(f"router {shape.name} T={T}", flush=True)
    rng = np.random.default_rng(17)
    W = synth.make_router(rng, shape.n_experts, shape.hidden, std=0.02)
    x = synth.make_x(rng, T, shape.hidden)
    kind = moe.ROUTER_SOFTMAX if shape.router == "softmax" else moe.ROUTER_SIGMOID
    dW, dx = to_device(W), to_device(x)
    lg = DeviceBuffer(4 * T * shape.n_experts)
    di, dw = DeviceBuffer(4 * T * shape.top_k), DeviceBuffer(4 * T * shape.top_k)
    moe.moe_route(dW.ptr, 0, dx.ptr, T, shape.hidden, shape.n_experts, shape.top_k, kind,
                  lg.ptr, di.ptr, dw.ptr)
    synchronize()
    idx = di.download(np.int32, (T, shape.top_k))
    w = dw.download(np.float32, (T, shape.top_k))
    for t in range(T):
        oi, ow, _ = O.router_topk(W.view(np.uint16), None, x[t].astype(np.float32), shape.top_k,
                                  kind=shape.router)
        l = W.astype(np.float64) @ x[t].astype(np.float64)
        srt = np.sort(l)[::-1]
        gap = np.min(np.abs(np.diff(srt[: shape.top_k + 1])))
        if gap > 1e-4 * np.max(np.abs(l)):
            assert idx[t].tolist() == oi.tolist(), (t, idx[t], oi)
            assert np.allclose(w[t], ow, rtol=1e-4)
        else:
            # decided by a near-tie: still a top-k of the float64 logits
            # within the margin (the sigmoid is monotonic in the logit)
            assert_valid_topk(l, idx[t], shape.top_k, 1e-4 * np.max(np.abs(l)), f"token {t}")


@pytest.mark.parametrize("T,k,E", [(1, 8, 256), (4, 2, 8), (2048, 8, 256), (37, 6, 1000),
                                   (1, 1, 1), (8192, 8, 1024), (3000, 9, 257)])
def test_expert_offsets_bit_exact(T, k, E):
    print(f"offsets T={T} k={k} E={E}", flush=True)
    rng = np.random.default_rng(T * k)
    t = synth.zipf_topk(rng, T, E, k) if T > 100 else synth.uniform_topk(rng, T, E, k)
    if T > 2:
        t[1, 0] = -1
        t[2, 1] = E + 5     # out of range: skipped like the oracle
    n = T * k
    dt = to_device(t)
    dc, do, dord, dinv = (DeviceBuffer(4 * E), DeviceBuffer(4 * (E + 1)), DeviceBuffer(4 * n),
                          DeviceBuffer(4 * n))
    dord.upload(np.full(n, -1, np.int32))
    moe.expert_offsets(dt.ptr, T, k, E, dc.ptr, do.ptr, dord.ptr, dinv.ptr)
    synchronize()
    counts, offsets, order = O.expert_offsets(t, E)
    assert np.array_equal(dc.download(np.int32, E), counts)
    assert np.array_equal(do.download(np.int32, E + 1), offsets)
    nv = int(offsets[-1])
    got_order = dord.download(np.int32, n)
    assert np.array_equal(got_order[:nv], order[:nv])
    inv = dinv.download(np.int32, n)
    flat = t.reshape(-1)
    for p in range(n):
        if 0 <= flat[p] < E:
            assert got_order[inv[p]] == p
        else:
            assert inv[p] == -1


def test_gather_and_weighted_combine():
    rng = np.random.default_rng(23)
    T, k, E, hidden = 64, 8, 256, 7168
    t = synth.zipf_topk(rng, T, E, k)
    w = synth.route_weights(rng, T, k)
    x = synth.make_x(rng, T, hidden)
    counts, offsets, order = O.expert_offsets(t, E)
    n = T * k
    inv = np.empty(n, np.int32)
    inv[order] = np.arange(n, dtype=np.int32)
    dx, dord = to_device(x), to_device(order)
    xg = DeviceBuffer(2 * n * hidden)
    moe._ck(moe.lib().wisp_gpu_moe_gather(dx.ptr, dord.ptr, n, k, hidden, xg.ptr, None), "gather")
    y = rng.standard_normal((n, hidden)).astype(np.float32)
    dy, dinv, dw = to_device(y), to_device(inv), to_device(w)
    out = DeviceBuffer(4 * T * hidden)
    moe._ck(moe.lib().wisp_gpu_moe_scatter(dy.ptr, dinv.ptr, dw.ptr, T, k, hidden, 0, out.ptr,
                                           None), "scatter")
    synchronize()
    g = xg.download(np.uint16, (n, hidden))
    assert np.array_equal(g, x.view(np.uint16)[order // k])
    want = np.zeros((T, hidden), np.float64)
    for tt in range(T):
        for s in range(k):
            want[tt] += w[tt, s] * y[inv[tt * k + s]].astype(np.float64)
    got = out.download(np.float32, (T, hidden))
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
