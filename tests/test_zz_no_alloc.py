"""The layer decode entry point that allocates nothing
(wisp_gpu_moe_layer_decode_int4_noalloc) against the one with a caller
workspace (wisp_gpu_moe_layer_decode_int4), through the C ABI.

Both run the same kernels on the same inputs, so the selection, the scores
and the outputs must be bit-identical; every shape is called twice in a
row, the second time with fewer tokens, so the static workspace keeps the
first call's contents while the second runs.
"""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from tests.gpu_util import make_expert
from wisp_amd import _lib, moe, synth
from wisp_amd.hip import DeviceBuffer, synchronize, to_device

pytestmark = pytest.mark.gpu


def _noalloc(dW, kind, scores, idx, w, table, shared, layout, x, M, top_k, n_exp, out32, out16):
    rc = _lib.lib().wisp_gpu_moe_layer_decode_int4_noalloc(
        dW, None, kind, scores, idx, w, table, shared or None, ctypes.byref(layout), x,
        moe.DTYPE_F16, M, top_k, n_exp, 0, out32, out16, None)
    return rc


@pytest.mark.parametrize("hidden,inter,n_exp,top_k,kind,shared", [
    (7168, 256, 64, 8, moe.ROUTER_SIGMOID, True),    # K-split gate/up (hidden > 4096)
    (1024, 1024, 8, 2, moe.ROUTER_SOFTMAX, False),
])
def test_noalloc_matches_workspace_entry_point(hidden, inter, n_exp, top_k, kind, shared):
    print(f"noalloc: hidden={hidden} inter={inter} experts={n_exp} top-{top_k}", flush=True)
    seed = hidden + n_exp
    rng = np.random.default_rng(seed)
    blobs = [make_expert(seed, e, inter, hidden, 128) for e in range(n_exp)]
    arena = moe.ExpertArena(n_exp, inter, hidden, 128, lambda e, out: blobs[e], has_zeros=False)
    sh = None
    if shared:
        sb = make_expert(seed, 777, inter, hidden, 128)
        sh = DeviceBuffer(sb.nbytes + 16)
        sh.upload(sb, offset=8)
    shp = sh.ptr + 8 if shared else 0
    W = synth.make_router(rng, n_exp, hidden, std=0.05)
    dW = to_device(W)
    for M in (4, 1):          # the second call is smaller
        x = synth.make_x(rng, M, hidden)
        dx = to_device(x)
        res = []
        for which in ("workspace", "noalloc"):
            scores = DeviceBuffer(4 * M * n_exp)
            idx, w = DeviceBuffer(4 * M * top_k), DeviceBuffer(4 * M * top_k)
            out32, out16 = DeviceBuffer(4 * M * hidden), DeviceBuffer(2 * M * hidden)
            if which == "workspace":
                ws = DeviceBuffer(moe.decode_workspace_bytes(arena.layout, M, top_k, shared))
                moe.moe_layer_decode_int4(dW.ptr, 0, kind, scores.ptr, idx.ptr, w.ptr,
                                          arena.table.ptr, shp, arena.layout, dx.ptr, M, top_k,
                                          n_exp, ws, out32=out32.ptr, out16=out16.ptr)
            else:
                rc = _noalloc(dW.ptr, kind, scores.ptr, idx.ptr, w.ptr, arena.table.ptr, shp,
                              arena.layout, dx.ptr, M, top_k, n_exp, out32.ptr, out16.ptr)
                assert rc == 0, rc
            synchronize()
            res.append((scores.download(np.float32, (M, n_exp)),
                        idx.download(np.int32, (M, top_k)), w.download(np.float32, (M, top_k)),
                        out32.download(np.float32, (M, hidden)),
                        out16.download(np.uint16, (M, hidden))))
        assert moe.decode_status(None) == 0
        for a, b, name in zip(res[0], res[1], ("scores", "idx", "w", "out32", "out16")):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"M={M}: {name} differs"
        assert np.isfinite(res[1][3]).all()


def _scratch_bytes():
    """WISP_NOALLOC_SCRATCH_BYTES as include/wisp_amd.h defines it."""
    hdr = (Path(__file__).resolve().parents[1] / "include" / "wisp_amd.h").read_text()
    m = re.search(r"#define WISP_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", hdr)
    assert m, "WISP_NOALLOC_SCRATCH_BYTES not found"
    return int(m.group(1)) << int(m.group(2))


def test_noalloc_rejects_a_layer_beyond_its_scratch():
    """Mixtral-8x7B shape with 4 tokens of top-8: the workspace would be about
    29 MB, over the static array; rejected before any launch. The call passes
    placeholder pointers, so it is made only once the size is known to exceed
    the array the header declares."""
    print("noalloc: size rejection", flush=True)
    hdr = np.zeros(synth.blob_size(14336, 4096, 128), np.uint8)
    synth.write_header(hdr, 0, 0, 14336, 4096, 128)
    L = moe.layout_from_blob(hdr, has_zeros=False)
    need = moe.decode_workspace_bytes(L, 4, 8, False)
    assert need > _scratch_bytes(), (need, _scratch_bytes())
    fake = 0x1000
    rc = _noalloc(fake, moe.ROUTER_SOFTMAX, fake, fake, fake, fake, 0, L, fake, 4, 8, 8, fake, None)
    assert rc == 1
    # and within it, the DeepSeek-V3 layer for 4 tokens fits
    hdr = np.zeros(synth.blob_size(2048, 7168, 128), np.uint8)
    synth.write_header(hdr, 0, 0, 2048, 7168, 128)
    L = moe.layout_from_blob(hdr, has_zeros=False)
    assert moe.decode_workspace_bytes(L, 4, 8, True) <= _scratch_bytes()
