"""Bounded cross-workgroup waits of the fused decode report a give-up.

The host makes every wait give up on purpose (wisp_amd__test_decode_wait:
a poll limit of a few polls and a wait target raised out of reach), so every
kernel still exits normally; the status word must then carry the wait's
bit and the outputs it feeds must be NaN. With the defaults restored, the
same workspace gives clean results that match the oracle and a zero status.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import assert_close, make_expert
from wisp_amd import _lib, moe, synth
from wisp_amd.hip import DeviceBuffer, synchronize, to_device

pytestmark = pytest.mark.gpu


class _Setup:
    def __init__(self, seed, inter=256, hidden=512, n_exp=8, top_k=2, M=1, kind="softmax"):
        self.inter, self.hidden, self.n_exp, self.top_k, self.M = inter, hidden, n_exp, top_k, M
        rng = np.random.default_rng(seed)
        self.blobs = [make_expert(seed, e, inter, hidden, 128) for e in range(n_exp)]
        self.shared = make_expert(seed, 999, inter, hidden, 128)
        self.arena = moe.ExpertArena(n_exp, inter, hidden, 128, lambda e, out: self.blobs[e],
                                     has_zeros=False)
        self.sh = DeviceBuffer(self.shared.nbytes + 16)
        self.sh.upload(self.shared, offset=8)
        self.x = synth.make_x(rng, M, hidden)
        self.dx = to_device(self.x)
        self.W = synth.make_router(rng, n_exp, hidden, std=0.05)
        self.dW = to_device(self.W)
        self.kind = kind
        self.idx = synth.uniform_topk(rng, M, n_exp, top_k)
        self.w = synth.route_weights(rng, M, top_k)
        self.di, self.dw = to_device(self.idx), to_device(self.w)
        self.ws = DeviceBuffer(moe.decode_workspace_bytes(self.arena.layout, M, top_k, True))
        self.scores = DeviceBuffer(4 * M * n_exp)
        self.ridx, self.rw = DeviceBuffer(4 * M * top_k), DeviceBuffer(4 * M * top_k)
        self.out = DeviceBuffer(4 * M * hidden)

    def given(self):
        moe.moe_decode_int4(self.arena.table.ptr, self.sh.ptr + 8, self.arena.layout, self.dx.ptr,
                            self.M, self.di.ptr, self.dw.ptr, self.top_k, self.n_exp, self.ws,
                            out32=self.out.ptr)
        synchronize()
        return self.out.download(np.float32, (self.M, self.hidden))

    def layer(self):
        k = moe.ROUTER_SOFTMAX if self.kind == "softmax" else moe.ROUTER_SIGMOID
        moe.moe_layer_decode_int4(self.dW.ptr, 0, k, self.scores.ptr, self.ridx.ptr, self.rw.ptr,
                                  self.arena.table.ptr, self.sh.ptr + 8, self.arena.layout,
                                  self.dx.ptr, self.M, self.top_k, self.n_exp, self.ws,
                                  out32=self.out.ptr)
        synchronize()
        return self.out.download(np.float32, (self.M, self.hidden))

    def want_given(self, t):
        return O.moe_combine(self.blobs, self.shared, self.x[t].astype(np.float32), self.idx[t],
                             self.w[t])

    def want_layer(self, t):
        oi, ow, _ = O.router_topk(self.W.view(np.uint16), None, self.x[t].astype(np.float32),
                                  self.top_k, kind=self.kind)
        return O.moe_combine(self.blobs, self.shared, self.x[t].astype(np.float32), oi, ow)


def _force(limit, extra):
    _lib.lib().wisp_amd__test_decode_wait(limit, extra)


def test_down_wait_give_up_is_reported_and_poisons():
    """One token: gate/up and down share a launch; every down wave gives up
    waiting for its unit's h' after 4 polls."""
    print("decode status: forced down-wait give-up", flush=True)
    s = _Setup(11)
    try:
        _force(4, 1 << 20)
        got = s.given()
    finally:
        _force(0, 0)
    st = moe.decode_status(s.ws)
    assert st & moe.DECODE_DOWN_WAIT, st
    assert np.isnan(got).all()
    # cleared by the read above
    assert moe.decode_status(s.ws) == 0
    got = s.given()
    assert moe.decode_status(s.ws) == 0
    assert_close(got[0], s.want_given(0), "clean call after the give-up")


@pytest.mark.parametrize("kind", ["softmax", "sigmoid"])
def test_router_wait_give_up_is_reported_and_poisons(kind):
    """Routing in the prep launch: the prep workgroup gives up waiting for
    the router workgroups' logits; the selection weights and the output are
    NaN and both waits report (the down waits are forced too)."""
    print(f"decode status: forced router-wait give-up ({kind})", flush=True)
    s = _Setup(12, kind=kind)
    try:
        _force(4, 1 << 20)
        got = s.layer()
    finally:
        _force(0, 0)
    st = moe.decode_status(s.ws, clear=False)
    assert st & moe.DECODE_ROUTER_WAIT, st
    assert st & moe.DECODE_DOWN_WAIT, st
    assert np.isnan(s.rw.download(np.float32, (s.M, s.top_k))).all()
    assert np.isnan(got).all()
    assert moe.decode_status(s.ws) == st      # clear
    # the epoch advanced past the abandoned call: the next calls are clean
    for _ in range(2):
        got = s.layer()
        assert moe.decode_status(s.ws) == 0
        assert_close(got[0], s.want_layer(0), "clean layer call after the give-up")


def test_multi_token_status_stays_clear():
    """Two launches for M > 1 (no in-launch hand-off for the down kernel):
    normal calls leave the status at zero."""
    print("decode status: M=3 clean", flush=True)
    s = _Setup(13, M=3)
    got = s.layer()
    assert moe.decode_status(s.ws) == 0
    for t in range(3):
        assert_close(got[t], s.want_layer(t), f"token {t}")
