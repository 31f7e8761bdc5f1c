"""GPU: the decode step's operations around the MoE layer.

* The reference-named launchers (wisp_gpu_rmsnorm, wisp_gpu_residual_add,
  wisp_gpu_swiglu, wisp_gpu_gemv_t_f16) against the fixture written by the
  reference's own scalar C (tests/golden/layer_ops.npz) and against the
  oracle on other sizes, aligned and not (the scalar fallbacks).
* wisp_gpu_moe_block_int4, x += MoE(RMSNorm(x) * w) over n rows of the
  residual stream, against the oracle's composition (rmsnorm, router,
  run_moe, residual add): 1, 3 and 7 rows (the fused decode, fp32 routing,
  in calls of up to 4 rows), 4 rows as a speculative-verify batch checked
  against four one-row calls, and 9 and 40 rows (routing on fp16 rows, then
  the grouped GEMM).

Bars: fp32 elementwise ops within 1e-6 relative (the GPU sums in fp32, the
reference's RMSNorm in double); MoE outputs at tests/gpu_util.py's bar."""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import assert_close, make_expert
from wisp_amd import _lib, moe, synth
from wisp_amd.hip import DeviceBuffer, synchronize, to_device

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "layer_ops.npz")


def _block_decode_max_rows():
    """WISP_BLOCK_DECODE_MAX_ROWS as include/wisp_amd.h defines it."""
    hdr = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                       "wisp_amd.h")
    import re
    with open(hdr) as f:
        m = re.search(r"#define WISP_BLOCK_DECODE_MAX_ROWS (\d+)", f.read())
    assert m, "WISP_BLOCK_DECODE_MAX_ROWS not found"
    return int(m.group(1))


BLOCK_DECODE_MAX_ROWS = _block_decode_max_rows()


def _close(got, want, rel=1e-6, what=""):
    err = np.max(np.abs(np.asarray(got, np.float64) - want)) / max(np.max(np.abs(want)), 1e-30)
    assert err <= rel, f"{what}: rel err {err:.2e}"


def test_reference_launchers_vs_golden():
    print("layer ops: golden", flush=True)
    g = np.load(GOLD)
    L = _lib.lib()
    n = g["x"].size
    dx, dw, dy = to_device(g["x"]), to_device(g["w"]), DeviceBuffer(4 * n)
    L.wisp_gpu_rmsnorm(dx.ptr, dw.ptr, dy.ptr, n, float(g["eps"]), None)
    rows, cols = g["Wt"].shape
    dW, dxt, dyt = to_device(g["Wt"]), to_device(g["xt"]), DeviceBuffer(4 * cols)
    L.wisp_gpu_gemv_t_f16(dW.ptr, dxt.ptr, dyt.ptr, rows, cols, None)
    dr, dd = to_device(g["r0"]), to_device(g["d"])
    L.wisp_gpu_residual_add(dr.ptr, dd.ptr, n, None)
    synchronize()
    _close(dy.download(np.float32, n), g["y"], what="rmsnorm")
    _close(dyt.download(np.float32, cols), g["yt"], what="gemv_t")
    assert np.array_equal(dr.download(np.float32, n), g["r1"])


@pytest.mark.parametrize("n", [1, 7, 1001, 4096, 7168, 20000])
def test_rmsnorm_residual_swiglu_vs_oracle(n):
    print(f"layer ops: n={n}", flush=True)
    rng = np.random.default_rng(n)
    L = _lib.lib()
    x = (rng.standard_normal(n) * 2).astype(np.float32)
    w = (1 + 0.2 * rng.standard_normal(n)).astype(np.float16)
    dx, dw = to_device(x), to_device(w)
    L.wisp_gpu_rmsnorm(dx.ptr, dw.ptr, dx.ptr, n, 1e-5, None)      # in place
    g, u = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    dg, du, do = to_device(g), to_device(u), DeviceBuffer(4 * n)
    L.wisp_gpu_swiglu(dg.ptr, du.ptr, do.ptr, n, None)
    r = rng.standard_normal(n).astype(np.float32)
    dr = to_device(r)
    L.wisp_gpu_residual_add(dr.ptr, dg.ptr, n, None)
    L.wisp_gpu_rmsnorm(dx.ptr, dw.ptr, dx.ptr, 0, 1e-5, None)       # early return
    synchronize()
    _close(dx.download(np.float32, n), O.rmsnorm(x, w, 1e-5), what="rmsnorm")
    want = np.empty(n, np.float32)
    O.orc().orc_swiglu(O._p(g), O._p(u), O._p(want), n)
    _close(do.download(np.float32, n), want, rel=2e-6, what="swiglu")
    assert np.array_equal(dr.download(np.float32, n), O.residual_add(r, g))


@pytest.mark.parametrize("rows,cols", [(96, 512), (33, 70), (7168, 2048), (130, 7168)])
def test_gemv_t_vs_oracle(rows, cols):
    print(f"layer ops: gemv_t {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows + cols)
    W = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float16)
    x = rng.standard_normal(rows).astype(np.float32)
    dW, dx, dy = to_device(W), to_device(x), DeviceBuffer(4 * cols)
    _lib.lib().wisp_gpu_gemv_t_f16(dW.ptr, dx.ptr, dy.ptr, rows, cols, None)
    synchronize()
    _close(dy.download(np.float32, cols), O.gemv_t_f16(W, x), rel=1e-5, what="gemv_t")


class _Block:
    def __init__(self, seed, hidden=7168, inter=256, n_exp=64, top_k=8, kind="sigmoid"):
        self.hidden, self.inter, self.n_exp, self.top_k, self.kind = hidden, inter, n_exp, top_k, kind
        rng = np.random.default_rng(seed)
        self.blobs = [make_expert(seed, e, inter, hidden, 128) for e in range(n_exp)]
        self.shared = make_expert(seed, 5000, inter, hidden, 128)
        self.arena = moe.ExpertArena(n_exp, inter, hidden, 128, lambda e, out: self.blobs[e],
                                     has_zeros=False)
        self.sh = DeviceBuffer(self.shared.nbytes + 16)
        self.sh.upload(self.shared, offset=8)
        self.W = synth.make_router(rng, n_exp, hidden, std=0.05)
        self.dW = to_device(self.W)
        self.norm_w = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float16)
        self.dnw = to_device(self.norm_w)
        self.rng = rng
        self.code = moe.ROUTER_SOFTMAX if kind == "softmax" else moe.ROUTER_SIGMOID

    def run(self, x):
        M = x.shape[0]
        dx = to_device(x)
        scores = DeviceBuffer(4 * M * self.n_exp)
        idx, w = DeviceBuffer(4 * M * self.top_k), DeviceBuffer(4 * M * self.top_k)
        ws = DeviceBuffer(moe.block_workspace_bytes(self.arena.layout, M, self.top_k, self.n_exp,
                                                    True))
        moe.moe_block_int4(dx.ptr, self.dnw.ptr, 1e-6, self.dW.ptr, 0, self.code, scores.ptr,
                           idx.ptr, w.ptr, self.arena.table.ptr, self.sh.ptr + 8,
                           self.arena.layout, M, self.top_k, self.n_exp, ws)
        synchronize()
        if M <= BLOCK_DECODE_MAX_ROWS:
            assert moe.decode_status(ws) == 0
        return (dx.download(np.float32, x.shape), idx.download(np.int32, (M, self.top_k)),
                w.download(np.float32, (M, self.top_k)))

    def want(self, x_row, fp16_route, dev_idx, dev_w):
        xn = O.rmsnorm(x_row, self.norm_w, 1e-6)
        xr = xn.astype(np.float16).astype(np.float32) if fp16_route else xn
        oi, ow, _ = O.router_topk(self.W.view(np.uint16), None, xr, self.top_k, kind=self.kind)
        if oi.tolist() != dev_idx.tolist():
            # only a near-tie of the fp32 keys may differ: check the device's choice
            l = self.W.astype(np.float64) @ xr.astype(np.float64)
            key = 1 / (1 + np.exp(-l)) if self.kind == "sigmoid" else l
            srt = np.sort(key)[::-1][: self.top_k + 1]
            assert np.min(np.abs(np.diff(srt))) <= 2e-5 * max(np.max(np.abs(srt)), 1.0), \
                (oi, dev_idx)
            oi, ow = dev_idx, dev_w
        ffn = O.moe_combine(self.blobs, self.shared, xn, oi, ow, fast=True)
        return x_row + ffn, ffn


@pytest.mark.parametrize("M", [1, 3, 7, 9, 40])
def test_moe_block_matches_oracle_composition(M):
    print(f"moe block: {M} rows", flush=True)
    b = _Block(600 + M)
    x = (b.rng.standard_normal((M, b.hidden)) * 1.5).astype(np.float32)
    got, gi, gw = b.run(x)
    for t in range(M):
        want, ffn = b.want(x[t], M > BLOCK_DECODE_MAX_ROWS, gi[t], gw[t])
        assert_close(got[t] - x[t], ffn, f"row {t}: the added ffn")


def test_verify_batch_equals_single_rows():
    """Speculative verify of 4 drafted tokens: one 4-row call gives each
    row what a one-row call gives it (to the fp16 bar: the 4-row and 1-row
    kernels sum in other orders)."""
    print("moe block: verify batch of 4", flush=True)
    b = _Block(77, kind="softmax", n_exp=32, top_k=4)
    x = (b.rng.standard_normal((4, b.hidden))).astype(np.float32)
    batch, bi, _ = b.run(x)
    for t in range(4):
        one, oi, _ = b.run(x[t:t + 1].copy())
        assert oi[0].tolist() == bi[t].tolist()
        assert_close(batch[t] - x[t], one[0] - x[t], f"row {t} batch vs one")


def test_block_rejects_bad_arguments():
    b = _Block(5, n_exp=8, top_k=2, inter=128, hidden=512)
    ws = DeviceBuffer(64)
    d = DeviceBuffer(4 * 512)
    with pytest.raises(Exception):   # workspace too small
        moe.moe_block_int4(d.ptr, b.dnw.ptr, 1e-6, b.dW.ptr, 0, b.code, d.ptr, d.ptr, d.ptr,
                           b.arena.table.ptr, 0, b.arena.layout, 1, 2, 8, ws)
    with pytest.raises(Exception):   # no rows
        moe.moe_block_int4(d.ptr, b.dnw.ptr, 1e-6, b.dW.ptr, 0, b.code, d.ptr, d.ptr, d.ptr,
                           b.arena.table.ptr, 0, b.arena.layout, 0, 2, 8, DeviceBuffer(1 << 20))
