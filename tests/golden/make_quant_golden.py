"""Writes tests/golden/quantize_int4.npz: inputs and outputs of the reference
converter's quantize_int4 / dequantize_int4 (wisp/converter/quantizer.py:
46-105), run from the reference tree in this container.

Only an import of the reference pins these bytes: quantize_int4 is torch
arithmetic (fp32 max/min, (max + min) / 2, (max - min) / 15 clamped at
1e-8, fp32 divide, torch.round half-to-even, clamp to 0..15, fp16 casts of
scale and zero), and the fixtures record what that arithmetic gives on
cases chosen to exercise it: half-way ties, constant groups (the clamp),
padded and odd-length matrices, groups that span rows, bf16 and fp16
inputs, and magnitudes whose fp16 scale or zero under- or overflows.

The module file is loaded on its own (it needs only torch), not through
the reference package, whose __init__ imports the downloader.

Usage: python tests/golden/make_quant_golden.py
Needs: the reference tree at /root/reference and torch (CPU).
"""
import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
QUANTIZER = "/root/reference/wisp/converter/quantizer.py"


def load_reference_quantizer():
    spec = importlib.util.spec_from_file_location("reference_quantizer", QUANTIZER)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod      # dataclasses look the module up by name
    spec.loader.exec_module(mod)
    return mod


def cases():
    """(name, weight tensor, group_size)."""
    g = torch.Generator().manual_seed(20261202)
    out = []
    # plain fp32 weights at a real model's scale, groups within rows
    out.append(("f32_normal", torch.randn(64, 256, generator=g) * 0.02, 128))
    # bf16 and fp16 checkpoints (converted to fp32 inside quantize_int4)
    out.append(("bf16_normal", (torch.randn(48, 384, generator=g) * 0.05).to(torch.bfloat16), 64))
    out.append(("f16_normal", (torch.randn(40, 512, generator=g) * 0.02).to(torch.float16), 128))
    # ties: a group holding the integers 0..15 has zero 7.5 and scale 1, so
    # every (x - zero) / scale is a half-integer and rounds to even
    w = torch.randn(8, 128, generator=g)
    w[0, :64] = torch.arange(64, dtype=torch.float32) % 16
    w[1, :64] = (torch.arange(64, dtype=torch.float32) % 16) * 0.25 - 2.0
    # constant groups (scale clamps to 1e-8), an all-zero group, a group of
    # two values
    w[2, :64] = 1.0
    w[2, 64:] = 0.0
    w[3, :64] = torch.where(torch.arange(64) % 2 == 0, torch.tensor(-3.0), torch.tensor(5.0))
    # tiny ranges: the fp16 scale goes subnormal or below the clamp
    w[4, :64] = 1e-3 + torch.randn(64, generator=g) * 1e-9
    w[4, 64:] = torch.randn(64, generator=g) * 1e-6
    # large magnitudes: the fp16 zero overflows to inf in one group
    w[5, :64] = 9.0e4 + torch.rand(64, generator=g) * 1.0e4
    w[5, 64:] = torch.randn(64, generator=g) * 3.0e4
    out.append(("f32_special_g64", w, 64))
    # odd element count (the last group is padded with the last element and
    # the last byte's high nibble is 0) and groups that span rows
    out.append(("f32_odd_3x43_g128", torch.randn(3, 43, generator=g), 128))
    out.append(("f32_span_6x100_g64", torch.randn(6, 100, generator=g) * 0.1, 64))
    # a blob shape the kernels read (inter 128, hidden 256, g128)
    for name, (r, c) in (("gate", (128, 256)), ("up", (128, 256)), ("down", (256, 128))):
        out.append((f"expert_{name}", torch.randn(r, c, generator=g) * 0.03, 128))
    return out


def main():
    q = load_reference_quantizer()
    arrays = {}
    names = []
    for name, w, gs in cases():
        qt = q.quantize_int4(w, group_size=gs)
        dq = q.dequantize_int4(qt)
        names.append(name)
        if w.dtype == torch.bfloat16:
            arrays[f"{name}/w_bf16"] = w.view(torch.int16).numpy().view(np.uint16)
        elif w.dtype == torch.float16:
            arrays[f"{name}/w_f16"] = w.numpy().view(np.uint16)
        else:
            arrays[f"{name}/w_f32"] = w.numpy()
        arrays[f"{name}/gs"] = np.int64(gs)
        arrays[f"{name}/packed"] = qt.packed.numpy()
        arrays[f"{name}/scales"] = qt.scales.numpy().view(np.uint16)
        arrays[f"{name}/zeros"] = qt.zeros.numpy().view(np.uint16)
        arrays[f"{name}/dequant_f16"] = dq.numpy().view(np.uint16)
    arrays["names"] = np.array(names)
    path = os.path.join(HERE, "quantize_int4.npz")
    np.savez_compressed(path, **arrays)
    print("wrote", path, "cases:", ", ".join(names))


if __name__ == "__main__":
    main()
