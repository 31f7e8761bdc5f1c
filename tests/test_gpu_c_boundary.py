"""The C-ABI boundary exercised from C (tests/c_abi/engine_call_shape.c,
compiled with gcc -std=c11 -Werror against include/wisp_amd.h, with the
reference's own launcher declarations repeated as written).

From C it runs the reference engine's per-expert sequence gpu_expert_ffn
(csrc/core/wisp_engine.c:1507-1531) and one fused layer call; the results
are checked against the golden fixtures written by the reference's own
compiled C (tests/golden/) and against the oracle."""
import ctypes
import os
from ctypes import c_float, c_int, c_size_t, c_void_p

import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import assert_close
from wisp_amd import _lib, moe, synth

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
CLIB = os.path.join(HERE, "c_abi", "libengine_call_shape.so")


def clib():
    _lib.lib()   # the product library first (RTLD_GLOBAL), as the engine would link it
    if not os.path.exists(CLIB):
        raise OSError(f"{CLIB} is not built; run __graft_entry__.build()")
    h = ctypes.CDLL(CLIB)
    h.c_gpu_expert_ffn.restype = c_int
    h.c_gpu_expert_ffn.argtypes = [c_void_p, c_size_t, c_void_p, c_float, c_void_p]
    h.c_moe_layer_decode.restype = c_int
    h.c_moe_layer_decode.argtypes = [c_void_p, c_size_t, c_int, c_int, c_void_p, c_void_p, c_int,
                                     c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p]
    return h


def test_reference_expert_sequence_from_c():
    print("C boundary: gpu_expert_ffn sequence", flush=True)
    g = np.load(os.path.join(GOLD, "expert_ffn.npz"))
    blob = np.ascontiguousarray(g["blob"])
    x = np.ascontiguousarray(g["x"], np.float32)
    acc = np.ascontiguousarray(g["acc"], np.float32).copy()
    rc = clib().c_gpu_expert_ffn(blob.ctypes.data, blob.nbytes, x.ctypes.data, float(g["w"]),
                                 acc.ctypes.data)
    assert rc == 0, rc
    assert_close(acc - g["acc"], g["out"] - g["acc"], "C gpu_expert_ffn vs reference CPU")


def test_fused_layer_from_c_matches_reference_router_and_oracle():
    """64 experts (inter 256, hidden 512, g128, zeros), the softmax router of
    the golden fixture (bias included, top-8): the selection must equal the
    reference's cpu_router_topk output and the layer output the oracle's."""
    print("C boundary: fused layer call", flush=True)
    g = np.load(os.path.join(GOLD, "router_softmax.npz"))
    n_exp, hidden = g["W"].shape
    k = int(g["k"])
    inter, gs = 256, 128
    blobs = [synth.make_blob(np.random.default_rng([4242, e]), inter, hidden, gs, expert=e,
                             zeros=True) for e in range(n_exp)]
    size = blobs[0].nbytes
    host = np.ascontiguousarray(np.concatenate(blobs))
    W = np.ascontiguousarray(g["W"])
    bias = np.ascontiguousarray(g["bias"])
    x = np.ascontiguousarray(g["x"], np.float32)
    idx = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    out = np.empty(hidden, np.float32)
    rc = clib().c_moe_layer_decode(host.ctypes.data, size, n_exp, 1, W.ctypes.data,
                                   bias.ctypes.data, moe.ROUTER_SOFTMAX, x.ctypes.data, 1, k,
                                   idx.ctypes.data, w.ctypes.data, out.ctypes.data)
    assert rc == 0, rc
    assert idx.tolist() == g["idx"].tolist()
    assert np.allclose(w, g["w"], rtol=1e-5, atol=0)
    want = O.moe_combine(blobs, None, x, g["idx"], g["w"])
    assert_close(out, want, "C fused layer vs oracle")
