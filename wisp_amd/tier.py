"""Host-side mirror of the VRAM tier of the expert cache (include/wisp_amd.h
section 6): the policy alone and the tier with its device memory, over the
C-ABI."""
from __future__ import annotations

import ctypes
import os

import numpy as np

from ._lib import lib
from .hip import check

VRAM_HIT, RAM_SCRATCH, RAM_PROMOTE, COLD_VRAM, COLD_SCRATCH = 0, 1, 2, 3, 4
STAT_NAMES = ("lookups", "vram_hits", "ram_hits", "first_touch", "promotions", "evictions",
              "scratch_serves", "h2d_bytes", "ram_evictions", "ssd_bytes", "d2h_bytes")
PROMOTE_HITS = 3   # the reference's WISP_PROMOTE_HITS


class Policy:
    """The tier policy alone (host only, no device calls)."""

    def __init__(self, n_layers: int, n_experts: int, n_slots: int, scratch_slots: int,
                 promote_hits: int = PROMOTE_HITS, n_ram_slots: int | None = None):
        """n_ram_slots None: every expert sits in RAM; else a RAM tier of
        that many blobs over the expert files (SSD tier)."""
        if n_ram_slots is None:
            self._h = lib().wisp_tier_policy_create(n_layers, n_experts, n_slots, scratch_slots,
                                                    promote_hits)
        else:
            self._h = lib().wisp_tier_policy_create_ram(n_layers, n_experts, n_ram_slots,
                                                        n_slots, scratch_slots, promote_hits)
        if not self._h:
            raise ValueError("wisp_tier_policy_create rejected its arguments")

    def begin_layer(self) -> None:
        lib().wisp_tier_policy_begin_layer(self._h)

    def lookup(self, layer: int, expert: int):
        """(path, slot, victim (layer, expert) or None)."""
        slot, vl, ve = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        path = lib().wisp_tier_policy_lookup(self._h, layer, expert, ctypes.byref(slot),
                                             ctypes.byref(vl), ctypes.byref(ve))
        if path < 0:
            raise ValueError(f"wisp_tier_policy_lookup({layer}, {expert})")
        return path, slot.value, (vl.value, ve.value) if vl.value >= 0 else None

    def stats(self) -> dict:
        out = (ctypes.c_uint64 * len(STAT_NAMES))()
        lib().wisp_tier_policy_stats(self._h, out)
        return dict(zip(STAT_NAMES, list(out)))

    def __del__(self):
        try:
            if self._h:
                lib().wisp_tier_policy_destroy(self._h)
        except Exception:
            pass


class ExpertTier:
    """VRAM slots + scratch ring over pinned host blobs (host_ptrs: list of
    pinned host addresses, layer-major)."""

    def __init__(self, n_layers: int, n_experts: int, blob_bytes: int, host_ptrs,
                 n_slots: int, scratch_slots: int, promote_hits: int = PROMOTE_HITS,
                 model_path: str | None = None, n_ram_slots: int = 0):
        """host_ptrs: pinned blobs of every expert (RAM tier holds all), or
        None with model_path and n_ram_slots: a bounded RAM tier over the
        expert files (wisp_tier_create_ssd)."""
        self.n_layers, self.n_experts = n_layers, n_experts
        err = ctypes.c_int(0)
        if host_ptrs is not None:
            self._ptrs = (ctypes.c_void_p * (n_layers * n_experts))(*host_ptrs)
            self._h = lib().wisp_tier_create(n_layers, n_experts, blob_bytes, self._ptrs, n_slots,
                                             scratch_slots, promote_hits, ctypes.byref(err))
        else:
            self._h = lib().wisp_tier_create_ssd(n_layers, n_experts, blob_bytes,
                                                 os.fsencode(model_path), n_ram_slots, n_slots,
                                                 scratch_slots, promote_hits, ctypes.byref(err))
        if not self._h:
            check(err.value or 1, "wisp_tier_create")

    def table(self, layer: int) -> int:
        return lib().wisp_tier_device_table(self._h, layer) or 0

    def fetch_layer(self, layer: int, expert_ids, compute: int = 0) -> np.ndarray:
        ids = np.ascontiguousarray(expert_ids, dtype=np.int32).reshape(-1)
        paths = np.empty(ids.size, np.int32)
        check(lib().wisp_tier_fetch_layer(self._h, layer, ids.ctypes.data, ids.size,
                                          paths.ctypes.data, compute or None), "wisp_tier_fetch_layer")
        return paths

    def wait_copies(self, compute: int = 0) -> None:
        check(lib().wisp_tier_wait_copies(self._h, compute or None), "wisp_tier_wait_copies")

    def release_layer(self, compute: int = 0) -> None:
        check(lib().wisp_tier_release_layer(self._h, compute or None), "wisp_tier_release_layer")

    def moe_decode_layer(self, layer: int, shared_blob: int, layout, x: int, n_tokens: int,
                         topk_idx, topk_w, ws, out32: int, out16: int = 0, compute: int = 0,
                         x_dtype: int = 0) -> None:
        """One MoE decode layer with host-side routing ([n_tokens, top_k])."""
        idx = np.ascontiguousarray(topk_idx, dtype=np.int32)
        w = np.ascontiguousarray(topk_w, dtype=np.float32)
        top_k = idx.shape[-1]
        check(lib().wisp_tier_moe_decode_layer(self._h, layer, shared_blob or None,
                                               ctypes.byref(layout), x, x_dtype, n_tokens,
                                               idx.ctypes.data, w.ctypes.data, top_k, ws.ptr,
                                               ws.nbytes, out32 or None, out16 or None,
                                               compute or None), "wisp_tier_moe_decode_layer")

    def stats(self) -> dict:
        out = (ctypes.c_uint64 * len(STAT_NAMES))()
        lib().wisp_tier_stats(self._h, out)
        return dict(zip(STAT_NAMES, list(out)))

    def close(self) -> None:
        if self._h:
            lib().wisp_tier_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
