"""Host-side mirror of the real-weight ingestion functions (include/wisp_amd.h
section 7): the converter's int4 quantizer, the expert blob writer and the
expert file reader/writer, over the C-ABI."""
from __future__ import annotations

import ctypes
import os

import numpy as np

from ._lib import lib

WEIGHT_F32, WEIGHT_F16, WEIGHT_BF16 = 0, 1, 2
IO_BAD_ARGUMENT, IO_MISSING, IO_TOO_LARGE, IO_SHORT_READ = -1, -2, -3, -4


def _dtype_code(w: np.ndarray, bf16: bool) -> int:
    if bf16:
        assert w.dtype == np.uint16, "bf16 weights are passed as their uint16 bits"
        return WEIGHT_BF16
    if w.dtype == np.float32:
        return WEIGHT_F32
    if w.dtype == np.float16:
        return WEIGHT_F16
    raise TypeError(f"unsupported weight dtype {w.dtype}")


def quantize_int4(w: np.ndarray, group_size: int, bf16: bool = False):
    """(packed u8, scales u16 bits, zeros u16 bits) of a 2-D weight matrix."""
    w = np.ascontiguousarray(w)
    rows, cols = w.shape
    n = rows * cols
    ng = (n + group_size - 1) // group_size if group_size > 0 else 1   # C rejects gs <= 0
    packed = np.empty((n + 1) // 2, np.uint8)
    scales = np.empty(ng, np.uint16)
    zeros = np.empty(ng, np.uint16)
    rc = lib().wisp_quantize_int4(w.ctypes.data, _dtype_code(w, bf16), rows, cols, group_size,
                                  packed.ctypes.data, scales.ctypes.data, zeros.ctypes.data)
    if rc != 0:
        raise ValueError(f"wisp_quantize_int4: {rc}")
    return packed, scales, zeros


def quantize_expert_blob(gate: np.ndarray, up: np.ndarray, down: np.ndarray, group_size: int,
                         layer: int = 0, expert: int = 0, bf16: bool = False) -> np.ndarray:
    """One expert's blob (the reference file format) from its three
    projections: gate/up [inter, hidden], down [hidden, inter]."""
    gate, up, down = (np.ascontiguousarray(a) for a in (gate, up, down))
    inter, hidden = gate.shape
    assert up.shape == (inter, hidden) and down.shape == (hidden, inter)
    assert gate.dtype == up.dtype == down.dtype
    rows = (ctypes.c_uint32 * 3)(inter, inter, hidden)
    cols = (ctypes.c_uint32 * 3)(hidden, hidden, inter)
    size = lib().wisp_expert_blob_bytes(rows, cols, group_size)
    out = np.empty(size, np.uint8)
    got = lib().wisp_expert_quantize_blob(gate.ctypes.data, up.ctypes.data, down.ctypes.data,
                                          _dtype_code(gate, bf16), inter, hidden, group_size,
                                          layer, expert, out.ctypes.data, size)
    if got != size:
        raise ValueError("wisp_expert_quantize_blob failed")
    return out


def expert_file_path(model_path: str, layer: int, expert: int) -> str:
    buf = ctypes.create_string_buffer(1200)
    if lib().wisp_expert_file_path(buf, len(buf), os.fsencode(model_path), layer, expert) != 0:
        raise ValueError("path too long")
    return buf.value.decode()


def write_expert_file(model_path: str, layer: int, expert: int, blob: np.ndarray) -> None:
    b = np.ascontiguousarray(blob, dtype=np.uint8)
    rc = lib().wisp_expert_file_write(os.fsencode(model_path), layer, expert, b.ctypes.data,
                                      b.nbytes)
    if rc != 0:
        raise OSError(f"wisp_expert_file_write: {rc}")


def read_expert_file(model_path: str, layer: int, expert: int, dst_ptr: int,
                     max_bytes: int) -> int:
    """Reads the expert file into the host buffer at dst_ptr; returns the
    byte count, or raises OSError with the WISP_IO_* code."""
    n = lib().wisp_expert_file_read(os.fsencode(model_path), layer, expert, dst_ptr, max_bytes)
    if n < 0:
        raise OSError(f"wisp_expert_file_read({layer}, {expert}): {n}")
    return int(n)
