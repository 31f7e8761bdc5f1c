"""Loads the in-tree libwisp_amd.so and declares its C-ABI signatures.

There is no fallback: if the library is missing or fails to load, every
entry point raises. Build it with `python -m wisp_amd.build`.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, Structure, c_char_p, c_float, c_int, c_size_t, c_uint32, c_uint64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libwisp_amd.so"
_LIB = None


class WispExpertLayout(Structure):
    _fields_ = [
        ("packed_off", c_uint64 * 3),
        ("scales_off", c_uint64 * 3),
        ("zeros_off", c_uint64 * 3),
        ("rows", c_uint32 * 3),
        ("cols", c_uint32 * 3),
        ("group_size", c_uint32),
        ("has_zeros", c_uint32),
        ("total_bytes", c_uint64),
    ]


P = c_void_p  # device / host pointers and streams are passed as raw addresses

_SIGS = {
    # section 1: reference launcher interface
    "launch_dequant_expert": (c_int, [P, P, P, P, c_int, c_int, P]),
    "async_load_expert": (c_int, [P, P, P, P, P, P, P, c_int, c_int, P]),
    "wisp_gpu_gemv_f16": (None, [P, P, P, c_int, c_int, P]),
    "wisp_gpu_swiglu_ffn": (None, [P, P, P, P, c_int, c_int, P]),
    "wisp_gpu_scale_accum": (None, [P, P, c_float, c_int, P]),
    "wisp_gpu_router_topk": (None, [P, P, P, P, c_int, c_int, c_int, P, P, P]),
    "wisp_gpu_gemv_t_f16": (None, [P, P, P, c_int, c_int, P]),
    "wisp_gpu_rmsnorm": (None, [P, P, P, c_int, c_float, P]),
    "wisp_gpu_residual_add": (None, [P, P, c_int, P]),
    "wisp_gpu_swiglu": (None, [P, P, P, c_int, P]),
    # section 2: layout
    "wisp_expert_layout_from_blob": (c_int, [P, c_size_t, POINTER(WispExpertLayout)]),
    "wisp_expert_layout_check": (c_int, [POINTER(WispExpertLayout)]),
    # section 3: routing
    "wisp_gpu_moe_route": (c_int, [P, P, P, c_int, c_int, c_int, c_int, c_int, P, P, P, P]),
    "wisp_gpu_topk_from_logits": (c_int, [P, P, c_int, c_int, c_int, c_int, P, P, P, P]),
    "wisp_gpu_expert_offsets": (c_int, [P, c_int, c_int, c_int, P, P, P, P, P]),
    "wisp_gpu_moe_gather": (c_int, [P, P, c_int, c_int, c_int, P, P]),
    "wisp_gpu_moe_scatter": (c_int, [P, P, P, c_int, c_int, c_int, c_int, P, P]),
    # section 4: fused decode
    "wisp_moe_decode_workspace_bytes": (c_size_t, [POINTER(WispExpertLayout), c_int, c_int, c_int]),
    "wisp_gpu_moe_decode_int4": (c_int, [P, P, POINTER(WispExpertLayout), P, c_int, c_int, P, P,
                                         c_int, c_int, P, c_size_t, c_int, P, P, P]),
    "wisp_gpu_moe_layer_decode_int4": (c_int, [P, P, c_int, P, P, P, P, P, POINTER(WispExpertLayout),
                                               P, c_int, c_int, c_int, c_int, P, c_size_t, c_int,
                                               P, P, P]),
    "wisp_moe_decode_status": (c_int, [P, P, P, c_int]),
    "wisp_moe_block_workspace_bytes": (c_size_t, [POINTER(WispExpertLayout), c_int, c_int, c_int,
                                                  c_int]),
    "wisp_gpu_moe_block_int4": (c_int, [P, P, c_float, P, P, c_int, P, P, P, P, P,
                                        POINTER(WispExpertLayout), c_int, c_int, c_int, P,
                                        c_size_t, P]),
    "wisp_gpu_moe_layer_decode_int4_noalloc": (c_int, [P, P, c_int, P, P, P, P, P,
                                                       POINTER(WispExpertLayout), P, c_int, c_int,
                                                       c_int, c_int, c_int, P, P, P]),
    # section 5: fused prefill
    "wisp_moe_prefill_workspace_bytes": (c_size_t, [POINTER(WispExpertLayout), c_int, c_int, c_int,
                                                    c_int]),
    "wisp_gpu_moe_prefill_int4": (c_int, [P, P, POINTER(WispExpertLayout), P, c_int, P, P, c_int,
                                          c_int, P, c_size_t, c_int, P, P, P]),
    # section 6: VRAM tier
    "wisp_tier_policy_create": (c_void_p, [c_int, c_int, c_int, c_int, c_int]),
    "wisp_tier_policy_create_ram": (c_void_p, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "wisp_tier_policy_destroy": (None, [P]),
    "wisp_tier_policy_begin_layer": (None, [P]),
    "wisp_tier_policy_lookup": (c_int, [P, c_int, c_int, P, P, P]),
    "wisp_tier_policy_stats": (None, [P, P]),
    "wisp_tier_create": (c_void_p, [c_int, c_int, c_size_t, P, c_int, c_int, c_int, P]),
    "wisp_tier_create_ssd": (c_void_p, [c_int, c_int, c_size_t, c_char_p, c_int, c_int, c_int,
                                        c_int, P]),
    "wisp_tier_destroy": (None, [P]),
    "wisp_tier_device_table": (c_void_p, [P, c_int]),
    "wisp_tier_fetch_layer": (c_int, [P, c_int, P, c_int, P, P]),
    "wisp_tier_wait_copies": (c_int, [P, P]),
    "wisp_tier_release_layer": (c_int, [P, P]),
    "wisp_tier_stats": (None, [P, P]),
    "wisp_tier_moe_decode_layer": (c_int, [P, c_int, P, POINTER(WispExpertLayout), P, c_int, c_int,
                                           P, P, c_int, P, c_size_t, P, P, P]),
    # section 7: real-weight ingestion
    "wisp_quantize_int4": (c_int, [P, c_int, c_uint32, c_uint32, c_uint32, P, P, P]),
    "wisp_expert_blob_bytes": (c_size_t, [P, P, c_uint32]),
    "wisp_expert_blob_write": (c_size_t, [P, c_size_t, c_uint32, c_uint32, c_uint32, P, P, P, P,
                                          P]),
    "wisp_expert_quantize_blob": (c_size_t, [P, P, P, c_int, c_uint32, c_uint32, c_uint32,
                                             c_uint32, c_uint32, P, c_size_t]),
    "wisp_expert_file_path": (c_int, [P, c_size_t, c_char_p, c_uint32, c_uint32]),
    "wisp_expert_file_read": (ctypes.c_int64, [c_char_p, c_uint32, c_uint32, P, c_size_t]),
    "wisp_expert_file_write": (c_int, [c_char_p, c_uint32, c_uint32, P, c_size_t]),
    # profiling
    "wisp_amd_set_kernel_events": (None, [P, c_int]),
    # internal test hook (not in the header): bounded-wait poll limit and target offset
    "wisp_amd__test_decode_wait": (None, [c_int, c_int]),
    "wisp_amd_version": (c_char_p, []),
}


def lib():
    """The loaded library (raises OSError if it is not built)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise OSError(f"{LIB_PATH} is not built; run `python -m wisp_amd.build`")
        h = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in _SIGS.items():
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _LIB = h
    return _LIB


def signatures() -> dict:
    return dict(_SIGS)
