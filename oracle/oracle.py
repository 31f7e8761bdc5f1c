"""ctypes front end of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Loads oracle/liboracle.so (the C restatement, always built) and, when it
was built in this tree, oracle/_ref/libwisp_ref.so (the reference's own
scalar CPU path compiled from its sources). Only tests/, the smoke check
and bench.py's cpu_baseline leg use this module.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_int, c_size_t, c_uint16, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_ORC = None
_REF = None


def _p(a: np.ndarray):
    return a.ctypes.data_as(c_void_p)


def build() -> None:
    import subprocess
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def orc():
    global _ORC
    if _ORC is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            build()
        h = ctypes.CDLL(str(path))
        h.orc_half_to_float.restype = c_float
        h.orc_half_to_float.argtypes = [c_uint16]
        h.orc_float_to_half.restype = c_uint16
        h.orc_float_to_half.argtypes = [c_float]
        h.orc_float_to_half_trunc.restype = c_uint16
        h.orc_float_to_half_trunc.argtypes = [c_float]
        h.orc_blob_size.restype = c_size_t
        h.orc_blob_size.argtypes = [c_uint32, c_uint32, c_uint32]
        h.orc_blob_parse.restype = c_int
        h.orc_blob_parse.argtypes = [c_void_p, c_size_t, c_void_p]
        h.orc_fast_isa.restype = c_int
        h.orc_num_threads.restype = c_int
        h.orc_fill_random_bytes.argtypes = [c_void_p, c_size_t, c_uint64]
        h.orc_gemv_int4.argtypes = [c_void_p] * 5 + [c_int] * 3
        h.orc_gemv_int4_fast.argtypes = [c_void_p] * 5 + [c_int] * 3
        h.orc_gemv_int4_f64.argtypes = [c_void_p] * 5 + [c_int] * 3
        h.orc_gemv_f16.argtypes = [c_void_p] * 3 + [c_int] * 2
        h.orc_swiglu.argtypes = [c_void_p] * 3 + [c_int]
        h.orc_gemv_t_f16.argtypes = [c_void_p] * 3 + [c_int] * 2
        h.orc_rmsnorm.argtypes = [c_void_p] * 3 + [c_int, c_float]
        h.orc_residual_add.argtypes = [c_void_p, c_void_p, c_int]
        h.orc_scale_accum.argtypes = [c_void_p, c_void_p, c_float, c_int]
        h.orc_expert_ffn.argtypes = [c_void_p] * 4 + [c_float, c_void_p]
        h.orc_expert_ffn_fast.argtypes = [c_void_p] * 4 + [c_float, c_void_p]
        h.orc_topk_select.argtypes = [c_void_p, c_int, c_int, c_void_p, c_void_p]
        h.orc_router_softmax_topk.argtypes = [c_void_p] * 4 + [c_int] * 3 + [c_void_p] * 2
        h.orc_router_sigmoid_topk.argtypes = [c_void_p] * 4 + [c_int] * 3 + [c_void_p] * 2
        h.orc_moe_combine.argtypes = [c_void_p] * 6 + [c_int, c_void_p, c_void_p]
        h.orc_expert_offsets.argtypes = [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]
        h.orc_unpack_int4.argtypes = [c_void_p, c_size_t, c_void_p]
        h.orc_pack_int4.argtypes = [c_void_p, c_size_t, c_void_p]
        h.orc_dequant_fp16.argtypes = [c_void_p] * 3 + [c_size_t, c_int, c_void_p]
        h.orc_dequant_f32.argtypes = [c_void_p] * 3 + [c_size_t, c_int, c_void_p]
        _ORC = h
    return _ORC


def ref_built() -> bool:
    """Whether oracle/_ref was built here (checks the file; loads nothing)."""
    return (HERE / "_ref" / "libwisp_ref.so").exists()


class LazyRef:
    """Attribute access loads the reference build on first use, so importing
    a test module maps nothing into the process."""

    def __getattr__(self, name):
        return getattr(ref(), name)


def ref():
    """The compiled reference CPU path, or None when it was not built here."""
    global _REF
    if _REF is None:
        path = HERE / "_ref" / "libwisp_ref.so"
        if not path.exists():
            return None
        h = ctypes.CDLL(str(path))
        h.ref_gemv_int4.argtypes = [c_void_p] * 5 + [c_int] * 3
        h.ref_gemv_f16.argtypes = [c_void_p] * 3 + [c_int] * 2
        h.ref_swiglu.argtypes = [c_void_p] * 3 + [c_int]
        h.ref_gemv_t_f16.argtypes = [c_void_p] * 3 + [c_int] * 2
        h.ref_rmsnorm.argtypes = [c_void_p] * 3 + [c_int, c_float]
        h.ref_residual_add.argtypes = [c_void_p, c_void_p, c_int]
        h.ref_router_topk.argtypes = [c_void_p] * 4 + [c_int] * 3 + [c_void_p] * 2
        h.ref_half_to_float.restype = c_float
        h.ref_half_to_float.argtypes = [c_uint16]
        h.ref_float_to_half.restype = c_uint16
        h.ref_float_to_half.argtypes = [c_float]
        h.ref_parse_header.restype = c_int
        h.ref_parse_header.argtypes = [c_void_p, c_size_t, c_void_p]
        h.ref_debug_probe.restype = c_int
        h.ref_debug_probe.argtypes = [ctypes.c_char_p, c_int, c_int, c_void_p]
        h.ref_expert_ffn.restype = c_int
        h.ref_expert_ffn.argtypes = [c_void_p, c_size_t, c_void_p, c_void_p, c_float]
        h.ref_selftest_lru.restype = c_int
        h.ref_tier_create.restype = c_void_p
        h.ref_tier_create.argtypes = [ctypes.c_char_p, c_int, c_int, c_size_t, c_size_t, c_size_t]
        h.ref_tier_fetch.restype = c_int
        h.ref_tier_fetch.argtypes = [c_void_p, c_uint32, c_uint32]
        h.ref_tier_stats.argtypes = [c_void_p, c_void_p]
        _REF = h
    return _REF


# ---------------------------------------------------------------------------
# numpy conveniences
# ---------------------------------------------------------------------------

class BlobMeta(ctypes.Structure):
    _fields_ = [("packed_off", c_uint64 * 3), ("scales_off", c_uint64 * 3),
                ("zeros_off", c_uint64 * 3), ("rows", c_uint32 * 3), ("cols", c_uint32 * 3),
                ("group_size", c_uint32), ("layer_id", c_uint32), ("expert_id", c_uint32),
                ("total_bytes", c_uint64)]


def parse_blob(blob: np.ndarray) -> BlobMeta:
    m = BlobMeta()
    rc = orc().orc_blob_parse(_p(blob), blob.nbytes, ctypes.byref(m))
    if rc != 0:
        raise ValueError(f"orc_blob_parse: {rc}")
    return m


def gemv_int4(packed, scales, zeros, x, rows, cols, gs, fast=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    f = orc().orc_gemv_int4_fast if fast else orc().orc_gemv_int4
    f(_p(packed), _p(scales), _p(zeros), _p(x), _p(y), rows, cols, gs)
    return y


def gemv_int4_f64(packed, scales, zeros, x, rows, cols, gs):
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty(rows, dtype=np.float64)
    orc().orc_gemv_int4_f64(_p(packed), _p(scales), _p(zeros), _p(x), _p(y), rows, cols, gs)
    return y


def expert_ffn(blob: np.ndarray, x: np.ndarray, acc: np.ndarray | None = None, w: float = 1.0,
               fast: bool = False) -> np.ndarray:
    m = parse_blob(blob)
    hidden, inter = int(m.rows[2]), int(m.rows[0])
    x = np.ascontiguousarray(x, dtype=np.float32)
    acc = np.zeros(hidden, np.float32) if acc is None else acc
    scratch = np.empty(3 * inter + hidden, np.float32)
    f = orc().orc_expert_ffn_fast if fast else orc().orc_expert_ffn
    f(_p(blob), ctypes.byref(m), _p(x), _p(acc), float(w), _p(scratch))
    return acc


def moe_combine(blobs: list, shared_blob, x, idx, w, fast: bool = False) -> np.ndarray:
    """One token: shared (w = 1) then routed experts in rank order. With
    fast=True each expert runs on the vectorised path (orc_expert_ffn_fast,
    itself checked against the scalar one), in the same order."""
    if fast:
        x32 = np.ascontiguousarray(x, dtype=np.float32)
        m = parse_blob(blobs[0] if blobs else shared_blob)
        out = np.zeros(int(m.rows[2]), np.float32)
        if shared_blob is not None:
            expert_ffn(shared_blob, x32, out, 1.0, fast=True)
        for e, we in zip(np.asarray(idx).reshape(-1), np.asarray(w).reshape(-1)):
            if e >= 0:
                expert_ffn(blobs[int(e)], x32, out, float(we), fast=True)
        return out
    m = parse_blob(blobs[0] if blobs else shared_blob)
    hidden, inter = int(m.rows[2]), int(m.rows[0])
    arr = (c_void_p * max(1, len(blobs)))(*[b.ctypes.data for b in blobs])
    x = np.ascontiguousarray(x, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty(hidden, np.float32)
    scratch = np.empty(3 * inter + hidden, np.float32)
    orc().orc_moe_combine(arr, ctypes.byref(m), None if shared_blob is None else _p(shared_blob),
                          _p(x), _p(idx), _p(w), len(idx), _p(out), _p(scratch))
    return out


def topk_select(scores: np.ndarray, k: int):
    s = np.ascontiguousarray(scores, dtype=np.float32)
    idx = np.empty(k, np.int32)
    val = np.empty(k, np.float32)
    orc().orc_topk_select(_p(s), len(s), k, _p(idx), _p(val))
    return idx, val


def router_topk(W, bias, x, top_k, kind="softmax"):
    n_experts, hidden = W.shape
    logits = np.empty(n_experts, np.float32)
    idx = np.empty(top_k, np.int32)
    w = np.empty(top_k, np.float32)
    f = orc().orc_router_softmax_topk if kind == "softmax" else orc().orc_router_sigmoid_topk
    f(_p(np.ascontiguousarray(W)), None if bias is None else _p(bias),
      _p(np.ascontiguousarray(x, dtype=np.float32)), _p(logits), n_experts, hidden, top_k,
      _p(idx), _p(w))
    return idx, w, logits


def expert_offsets(topk_idx: np.ndarray, n_experts: int):
    t = np.ascontiguousarray(topk_idx, dtype=np.int32)
    n_tokens, top_k = t.shape
    counts = np.empty(n_experts, np.int32)
    offsets = np.empty(n_experts + 1, np.int32)
    order = np.full(n_tokens * top_k, -1, np.int32)
    orc().orc_expert_offsets(_p(t), n_tokens, top_k, n_experts, _p(counts), _p(offsets), _p(order))
    return counts, offsets, order


def dequant_fp16(packed, scales, zeros, n, gs) -> np.ndarray:
    out = np.empty(n, np.uint16)
    orc().orc_dequant_fp16(_p(packed), _p(scales), _p(zeros), n, gs, _p(out))
    return out


def dequant_f32(packed, scales, zeros, n, gs) -> np.ndarray:
    out = np.empty(n, np.float32)
    orc().orc_dequant_f32(_p(packed), _p(scales), _p(zeros), n, gs, _p(out))
    return out


def random_bytes(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.uint8)
    orc().orc_fill_random_bytes(_p(out), n, seed)
    return out


def gemv_t_f16(W, x):
    rows, cols = W.shape
    y = np.empty(cols, np.float32)
    orc().orc_gemv_t_f16(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(x, dtype=np.float32)),
                         _p(y), rows, cols)
    return y


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    orc().orc_rmsnorm(_p(x), _p(np.ascontiguousarray(w)), _p(y), x.size, float(eps))
    return y


def residual_add(x, d):
    out = np.array(x, dtype=np.float32, copy=True)
    orc().orc_residual_add(_p(out), _p(np.ascontiguousarray(d, dtype=np.float32)), out.size)
    return out
