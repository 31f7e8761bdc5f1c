"""GPU parity of the reference-signature launchers (include/wisp_amd.h
section 1) against the CPU oracle and the reference-produced fixtures."""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import assert_close
from wisp_amd import _lib, synth
from wisp_amd.hip import DeviceBuffer, synchronize, to_device

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.mark.parametrize("gs,n,offset", [(128, 1 << 16, 0), (64, 4096, 8), (37, 4099, 1), (16, 4096, 0)])
def test_dequant_bit_exact(gs, n, offset):
    print(f"dequant gs={gs} n={n} offset={offset}", flush=True)
    rng = np.random.default_rng(gs + n)
    packed = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
    ng = (n + gs - 1) // gs
    scales = (np.abs(rng.standard_normal(ng)) * 0.01).astype(np.float16).view(np.uint16)
    zeros = (rng.standard_normal(ng) * 0.01).astype(np.float16).view(np.uint16)
    dp = DeviceBuffer(packed.nbytes + 16).upload(packed, offset)
    ds, dz = to_device(scales), to_device(zeros)
    out = DeviceBuffer(2 * n + 16)
    rc = _lib.lib().launch_dequant_expert(dp.ptr + offset, ds.ptr, dz.ptr, out.ptr, n, gs, None)
    assert rc == 0
    synchronize()
    got = out.download(np.uint16, n)
    assert np.array_equal(got, O.dequant_fp16(packed, scales, zeros, n, gs))


def test_dequant_golden_fixture():
    g = np.load(os.path.join(GOLD, "dequant_g64.npz"))
    n, gs = int(g["n"]), int(g["gs"])
    dp, ds, dz = to_device(g["packed"]), to_device(g["scales"]), to_device(g["zeros"])
    out = DeviceBuffer(2 * n)
    assert _lib.lib().launch_dequant_expert(dp.ptr, ds.ptr, dz.ptr, out.ptr, n, gs, None) == 0
    synchronize()
    assert np.array_equal(out.download(np.uint16, n), g["out_f16"])


@pytest.mark.parametrize("rows,cols", [(1000, 4096), (37, 1001), (64, 7168)])
def test_gemv_f16_and_swiglu(rows, cols):
    print(f"gemv_f16 rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(rows)
    Wg = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float16)
    Wu = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float16)
    x = rng.standard_normal(cols).astype(np.float32)
    dg, du, dx = to_device(Wg), to_device(Wu), to_device(x)
    y, h = DeviceBuffer(4 * rows), DeviceBuffer(4 * rows)
    L = _lib.lib()
    L.wisp_gpu_gemv_f16(dg.ptr, dx.ptr, y.ptr, rows, cols, None)
    L.wisp_gpu_swiglu_ffn(dg.ptr, du.ptr, dx.ptr, h.ptr, rows, cols, None)
    synchronize()
    g64 = Wg.astype(np.float64) @ x
    u64 = Wu.astype(np.float64) @ x
    assert np.max(np.abs(y.download(np.float32, rows) - g64)) <= 1e-5 * np.max(np.abs(g64))
    h64 = g64 / (1 + np.exp(-g64)) * u64
    assert np.max(np.abs(h.download(np.float32, rows) - h64)) <= 1e-5 * np.max(np.abs(h64))


def test_scale_accum_and_early_returns():
    rng = np.random.default_rng(3)
    n = 10007
    acc = rng.standard_normal(n).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    da, dx = to_device(acc), to_device(x)
    L = _lib.lib()
    L.wisp_gpu_scale_accum(da.ptr, dx.ptr, 0.3, n, None)
    L.wisp_gpu_scale_accum(da.ptr, dx.ptr, 0.3, 0, None)      # no-op
    L.wisp_gpu_gemv_f16(dx.ptr, dx.ptr, da.ptr, 0, 16, None)    # no-op
    synchronize()
    want = acc.astype(np.float64) + np.float32(0.3) * x.astype(np.float64)
    assert np.max(np.abs(da.download(np.float32, n) - want)) <= 1e-6 * np.max(np.abs(want))


def test_reference_call_shape_expert_ffn():
    """The reference's gpu_expert_ffn sequence (csrc/core/wisp_engine.c:
    1507-1531) on these launchers, blob at the reference's 8-mod-16 section
    alignment, against the fixture produced by the reference CPU path."""
    g = np.load(os.path.join(GOLD, "expert_ffn.npz"))
    blob, inter, hidden, gs = g["blob"], int(g["inter"]), int(g["hidden"]), int(g["gs"])
    db = to_device(blob)
    dq = [DeviceBuffer(2 * inter * hidden) for _ in range(3)]
    m = O.parse_blob(blob)
    L = _lib.lib()
    for i in range(3):
        n = int(m.rows[i] * m.cols[i])
        rc = L.launch_dequant_expert(db.ptr + m.packed_off[i], db.ptr + m.scales_off[i],
                                     db.ptr + m.zeros_off[i], dq[i].ptr, n, gs, None)
        assert rc == 0
    dx, dacc = to_device(g["x"]), to_device(g["acc"])
    h, y = DeviceBuffer(4 * inter), DeviceBuffer(4 * hidden)
    L.wisp_gpu_swiglu_ffn(dq[0].ptr, dq[1].ptr, dx.ptr, h.ptr, inter, hidden, None)
    L.wisp_gpu_gemv_f16(dq[2].ptr, h.ptr, y.ptr, hidden, inter, None)
    L.wisp_gpu_scale_accum(dacc.ptr, y.ptr, float(g["w"]), hidden, None)
    synchronize()
    got = dacc.download(np.float32, hidden)
    assert_close(got - g["acc"], g["out"] - g["acc"], "reference call shape")


def test_reference_router_topk_golden():
    g = np.load(os.path.join(GOLD, "router_softmax.npz"))
    n_exp, hidden = g["W"].shape
    k = int(g["k"])
    dW, db, dx = to_device(g["W"]), to_device(g["bias"]), to_device(g["x"])
    lg = DeviceBuffer(4 * n_exp)
    idx = np.full(k, -7, np.int32)
    w = np.zeros(k, np.float32)
    _lib.lib().wisp_gpu_router_topk(dW.ptr, db.ptr, dx.ptr, lg.ptr, n_exp, hidden, k,
                                    idx.ctypes.data, w.ctypes.data, None)
    synchronize()
    assert idx.tolist() == g["idx"].tolist()
    assert np.allclose(w, g["w"], rtol=1e-5)
    assert np.allclose(lg.download(np.float32, n_exp), g["probs"], rtol=1e-4, atol=1e-8)
