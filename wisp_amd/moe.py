"""Host-side mirror of the MoE expert-path interface over the C-ABI.

Thin Python wrappers that keep the launcher argument meaning of
include/wisp_amd.h; every call goes to libwisp_amd.so and raises on a HIP
error code. Device memory comes from wisp_amd.hip.
"""
from __future__ import annotations

import ctypes
from typing import Callable, Sequence

import numpy as np

from . import synth
from ._lib import WispExpertLayout, lib
from .hip import DeviceBuffer, HipError, check, to_device

ROUTER_SOFTMAX = 0
ROUTER_SIGMOID = 1
DTYPE_F16 = 0
DTYPE_F32 = 1


def _ck(rc: int, what: str) -> None:
    if rc != 0:
        check(rc, what)


def layout_from_blob(blob: np.ndarray, has_zeros: bool = True) -> WispExpertLayout:
    L = WispExpertLayout()
    rc = lib().wisp_expert_layout_from_blob(blob.ctypes.data, blob.nbytes, ctypes.byref(L))
    if rc != 0:
        raise ValueError(f"wisp_expert_layout_from_blob: {rc}")
    L.has_zeros = 1 if has_zeros else 0
    return L


class ExpertArena:
    """Experts of one layer resident in one device allocation.

    Expert e's blob sits at base + e * stride + 8, so every blob section is
    16-byte aligned (the 120-byte header leaves sections at 8 mod 16 of the
    blob base). `table` is the device array of blob pointers the fused
    launchers index by expert id.
    """

    def __init__(self, n_experts: int, inter: int, hidden: int, gs: int,
                 make: Callable[..., np.ndarray], has_zeros: bool = True,
                 keep_host: Sequence[int] = (), only: Sequence[int] | None = None):
        """make(e, out) writes expert e's blob into the reusable host buffer
        `out` and returns it. With `only`, just those experts are uploaded (the
        other slots stay unwritten and must not be routed to)."""
        self.n_experts, self.inter, self.hidden, self.gs = n_experts, inter, hidden, gs
        self.stride = synth.slot_stride(inter, hidden, gs)
        self.buf = DeviceBuffer(self.stride * n_experts)
        self.host = {}
        staging = np.empty(synth.blob_size(inter, hidden, gs), np.uint8)
        layout = None
        for e in (range(n_experts) if only is None else sorted(set(only))):
            blob = make(e, staging)
            if layout is None:
                layout = layout_from_blob(blob, has_zeros)
            self.buf.upload(blob, offset=e * self.stride + 8)
            if e in keep_host:
                self.host[e] = blob.copy()
        self.layout = layout
        ptrs = np.array([self.ptr(e) for e in range(n_experts)], dtype=np.uint64)
        self.table = to_device(ptrs)

    def ptr(self, e: int) -> int:
        return self.buf.ptr + e * self.stride + 8


def decode_workspace_bytes(layout: WispExpertLayout, n_tokens: int, top_k: int, has_shared: bool) -> int:
    return int(lib().wisp_moe_decode_workspace_bytes(ctypes.byref(layout), n_tokens, top_k,
                                                      1 if has_shared else 0))


def moe_decode_int4(table: int, shared_blob: int, layout: WispExpertLayout, x: int,
                    n_tokens: int, topk_idx: int, topk_w: int, top_k: int, n_experts: int,
                    ws: DeviceBuffer, out32: int = 0, out16: int = 0, stream: int = 0,
                    accumulate: bool = False, x_dtype: int = DTYPE_F16) -> None:
    rc = lib().wisp_gpu_moe_decode_int4(table, shared_blob or None, ctypes.byref(layout), x,
                                        x_dtype, n_tokens, topk_idx, topk_w, top_k, n_experts,
                                        ws.ptr, ws.nbytes, 1 if accumulate else 0,
                                        out32 or None, out16 or None, stream or None)
    _ck(rc, "wisp_gpu_moe_decode_int4")


def moe_layer_decode_int4(router_w: int, router_bias: int, kind: int, scores: int, idx: int,
                          w: int, table: int, shared_blob: int, layout: WispExpertLayout, x: int,
                          n_tokens: int, top_k: int, n_experts: int, ws: DeviceBuffer,
                          out32: int = 0, out16: int = 0, stream: int = 0,
                          accumulate: bool = False, x_dtype: int = DTYPE_F16) -> None:
    """Router + routed/shared experts of one MoE layer (M = 1..4 tokens)."""
    rc = lib().wisp_gpu_moe_layer_decode_int4(router_w, router_bias or None, kind, scores, idx, w,
                                              table, shared_blob or None, ctypes.byref(layout), x,
                                              x_dtype, n_tokens, top_k, n_experts, ws.ptr,
                                              ws.nbytes, 1 if accumulate else 0, out32 or None,
                                              out16 or None, stream or None)
    _ck(rc, "wisp_gpu_moe_layer_decode_int4")


def prefill_workspace_bytes(layout: WispExpertLayout, n_tokens: int, top_k: int, n_experts: int,
                            has_shared: bool) -> int:
    return int(lib().wisp_moe_prefill_workspace_bytes(ctypes.byref(layout), n_tokens, top_k,
                                                       n_experts, 1 if has_shared else 0))


def moe_prefill_int4(table: int, shared_blob: int, layout: WispExpertLayout, x: int,
                     n_tokens: int, topk_idx: int, topk_w: int, top_k: int, n_experts: int,
                     ws: DeviceBuffer, out32: int = 0, out16: int = 0, stream: int = 0,
                     accumulate: bool = False) -> None:
    """Grouped-GEMM MoE over any number of tokens (fp16 x)."""
    rc = lib().wisp_gpu_moe_prefill_int4(table, shared_blob or None, ctypes.byref(layout), x,
                                         n_tokens, topk_idx, topk_w, top_k, n_experts, ws.ptr,
                                         ws.nbytes, 1 if accumulate else 0, out32 or None,
                                         out16 or None, stream or None)
    _ck(rc, "wisp_gpu_moe_prefill_int4")


def moe_route(router_w: int, bias: int, x: int, n_tokens: int, hidden: int, n_experts: int,
              top_k: int, kind: int, logits: int, idx: int, w: int, stream: int = 0) -> None:
    rc = lib().wisp_gpu_moe_route(router_w, bias or None, x, n_tokens, hidden, n_experts, top_k,
                                  kind, logits, idx, w, stream or None)
    _ck(rc, "wisp_gpu_moe_route")


def topk_from_logits(logits: int, bias: int, n_tokens: int, n_experts: int, top_k: int,
                     kind: int, scores: int, idx: int, w: int, stream: int = 0) -> None:
    rc = lib().wisp_gpu_topk_from_logits(logits, bias or None, n_tokens, n_experts, top_k, kind,
                                         scores, idx, w, stream or None)
    _ck(rc, "wisp_gpu_topk_from_logits")


def expert_offsets(topk_idx: int, n_tokens: int, top_k: int, n_experts: int, counts: int,
                   offsets: int, order: int, inv: int, stream: int = 0) -> None:
    rc = lib().wisp_gpu_expert_offsets(topk_idx, n_tokens, top_k, n_experts, counts, offsets,
                                       order, inv, stream or None)
    _ck(rc, "wisp_gpu_expert_offsets")


DECODE_ROUTER_WAIT = 1
DECODE_DOWN_WAIT = 2


def decode_status(ws: DeviceBuffer | None, stream: int = 0, clear: bool = True) -> int:
    """Status bits of the bounded waits of the most recent decode call on
    `ws` (None: the no-alloc entry point's static workspace); waits for
    `stream`; 0 when every wait completed."""
    flags = ctypes.c_uint32(0)
    rc = lib().wisp_moe_decode_status(ws.ptr if ws is not None else None, stream or None,
                                      ctypes.byref(flags), 1 if clear else 0)
    _ck(rc, "wisp_moe_decode_status")
    return int(flags.value)


def block_workspace_bytes(layout: WispExpertLayout, n_tokens: int, top_k: int, n_experts: int,
                          has_shared: bool) -> int:
    return int(lib().wisp_moe_block_workspace_bytes(ctypes.byref(layout), n_tokens, top_k,
                                                     n_experts, 1 if has_shared else 0))


def moe_block_int4(x: int, post_norm_w: int, eps: float, router_w: int, router_bias: int,
                   kind: int, scores: int, idx: int, w: int, table: int, shared_blob: int,
                   layout: WispExpertLayout, n_tokens: int, top_k: int, n_experts: int,
                   ws: DeviceBuffer, stream: int = 0) -> None:
    """x += MoE(RMSNorm(x) * post_norm_w) for n_tokens fp32 rows (in place)."""
    rc = lib().wisp_gpu_moe_block_int4(x, post_norm_w, eps, router_w, router_bias or None, kind,
                                       scores, idx, w, table, shared_blob or None,
                                       ctypes.byref(layout), n_tokens, top_k, n_experts, ws.ptr,
                                       ws.nbytes, stream or None)
    _ck(rc, "wisp_gpu_moe_block_int4")
