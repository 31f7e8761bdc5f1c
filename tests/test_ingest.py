"""Real-weight ingestion on the CPU: the int4 quantizer against the
reference converter's own output (tests/golden/quantize_int4.npz, written
by tests/golden/make_quant_golden.py from wisp/converter/quantizer.py), the
reference's known-answer tests for the format (tests/test_adapters.py:
250-308 there), and the expert file round trip through the reader."""
import os

import numpy as np
import pytest

from oracle import oracle as O
from wisp_amd import ingest, synth
from wisp_amd.moe import layout_from_blob

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "quantize_int4.npz")


def _cases():
    g = np.load(GOLD)
    for name in g["names"]:
        name = str(name)
        if f"{name}/w_f32" in g:
            w, bf16 = g[f"{name}/w_f32"], False
        elif f"{name}/w_f16" in g:
            w, bf16 = g[f"{name}/w_f16"].view(np.float16), False
        else:
            w, bf16 = g[f"{name}/w_bf16"], True
        yield name, w, bf16, int(g[f"{name}/gs"]), g


@pytest.mark.parametrize("case", [c[0] for c in _cases()])
def test_quantizer_bytes_match_reference_converter(case):
    for name, w, bf16, gs, g in _cases():
        if name != case:
            continue
        packed, scales, zeros = ingest.quantize_int4(w, gs, bf16=bf16)
        assert np.array_equal(packed, g[f"{name}/packed"]), f"{name}: packed bytes"
        assert np.array_equal(scales, g[f"{name}/scales"]), f"{name}: fp16 scales"
        assert np.array_equal(zeros, g[f"{name}/zeros"]), f"{name}: fp16 zeros"
        # the reference's dequantize_int4 (fp32 (q - 8) s + z, then fp16)
        # equals the oracle's dequant (the reference GPU kernel's formula)
        n = w.shape[0] * w.shape[1]
        dq = O.dequant_fp16(packed, scales, zeros, n, gs)
        assert np.array_equal(dq, g[f"{name}/dequant_f16"].reshape(-1)), f"{name}: dequant"


def test_fixture_covers_ties_clamp_padding_and_overflow():
    """What the special case is there to exercise actually occurs in it."""
    g = np.load(GOLD)
    sc = g["f32_special_g64/scales"].view(np.float16)
    z = g["f32_special_g64/zeros"].view(np.float16)
    assert (sc == 0).any()                    # 1e-8 clamp rounds to fp16 zero
    assert np.isinf(z).any()                  # zero above the fp16 range
    assert (sc.view(np.uint16) & 0x7C00 == 0).any() and (sc > 0).any()   # a subnormal scale
    assert g["f32_odd_3x43_g128/packed"].size == (3 * 43 + 1) // 2


def test_constant_group_packs_to_0x88():
    """tests/test_adapters.py:262-267 of the reference: a constant group
    quantizes to nibble 8 (byte 0x88) and dequantizes to its value."""
    w = np.full((2, 64), 1.0, np.float32)
    packed, scales, zeros = ingest.quantize_int4(w, 64)
    assert (packed == 0x88).all()
    dq = O.dequant_fp16(packed, scales, zeros, w.size, 64).view(np.float16)
    assert np.array_equal(dq, np.full(w.size, 1.0, np.float16))


def test_roundtrip_error_within_half_a_step():
    """tests/test_adapters.py:250-259 of the reference: the reconstruction
    error is at most about half a quantization step, mean below 0.005."""
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((64, 128)) * 0.02).astype(np.float32)
    packed, scales, zeros = ingest.quantize_int4(w, 64)
    rec = O.dequant_f32(packed, scales, zeros, w.size, 64).reshape(w.shape)
    err = np.abs(w - rec)
    grp = w.reshape(-1, 64)
    step = (grp.max(1) - grp.min(1)) / 15
    assert err.max() <= step.max() * 0.51 + 1e-6
    assert err.mean() < 0.005


def test_rejects_bad_input():
    with pytest.raises(ValueError):
        ingest.quantize_int4(np.ones((4, 4), np.float32), 0)
    w = np.ones((4, 64), np.float32)
    w[1, 3] = np.inf
    with pytest.raises(ValueError):
        ingest.quantize_int4(w, 64)


def test_expert_blob_layout_and_file_round_trip(tmp_path):
    """The blob layout walk of the reference's tests/test_adapters.py:
    281-308 (120-byte header, sections tiling the file exactly), the
    library's header parser and the oracle's, and the reader."""
    rng = np.random.default_rng(7)
    inter, hidden, gs = 128, 256, 128
    gate = (rng.standard_normal((inter, hidden)) * 0.03).astype(np.float32)
    up = (rng.standard_normal((inter, hidden)) * 0.03).astype(np.float32)
    down = (rng.standard_normal((hidden, inter)) * 0.03).astype(np.float32)
    blob = ingest.quantize_expert_blob(gate, up, down, gs, layer=3, expert=42)
    assert blob.nbytes == synth.blob_size(inter, hidden, gs)
    hdr = np.frombuffer(blob[:24].tobytes(), "<u4")
    assert hdr.tolist() == [0x57455850, 1, 3, 42, gs, 3]
    L = layout_from_blob(blob)
    assert L.total_bytes == blob.nbytes
    m = O.parse_blob(blob)
    assert (m.layer_id, m.expert_id, m.group_size) == (3, 42, gs)
    # the sections are the quantizer's output, in order gate, up, down
    for i, mat in enumerate((gate, up, down)):
        p, s, z = ingest.quantize_int4(mat, gs)
        off = int(L.packed_off[i])
        assert np.array_equal(blob[off:off + p.size], p)
        so, zo = int(L.scales_off[i]), int(L.zeros_off[i])
        assert np.array_equal(blob[so:so + 2 * s.size].view(np.uint16), s)
        assert np.array_equal(blob[zo:zo + 2 * z.size].view(np.uint16), z)
    if O.ref_built():
        # the reference's own parser (rows, cols, packed and scale offsets, gs)
        out = np.zeros(14, np.uint64)
        assert O.LazyRef().ref_parse_header(O._p(blob), blob.nbytes, O._p(out)) == 0
        assert out[6:9].tolist() == list(L.packed_off) and out[9:12].tolist() == list(L.scales_off)
        assert int(out[12]) == gs
    # file round trip
    os.makedirs(tmp_path / "experts")
    ingest.write_expert_file(str(tmp_path), 3, 42, blob)
    path = ingest.expert_file_path(str(tmp_path), 3, 42)
    assert path.endswith("experts/L003_E00042.bin") and os.path.getsize(path) == blob.nbytes
    dst = np.zeros(blob.nbytes + 100, np.uint8)
    n = ingest.read_expert_file(str(tmp_path), 3, 42, dst.ctypes.data, dst.nbytes)
    assert n == blob.nbytes and np.array_equal(dst[:n], blob)
    with pytest.raises(OSError, match=str(ingest.IO_TOO_LARGE)):
        ingest.read_expert_file(str(tmp_path), 3, 42, dst.ctypes.data, blob.nbytes - 1)
    with pytest.raises(OSError, match=str(ingest.IO_MISSING)):
        ingest.read_expert_file(str(tmp_path), 3, 43, dst.ctypes.data, dst.nbytes)


def test_bf16_and_f16_inputs_equal_their_fp32_values():
    """quantize_int4 converts the checkpoint to fp32 first (quantizer.py:56),
    so an fp16 or bf16 matrix quantizes like its exact fp32 values."""
    rng = np.random.default_rng(3)
    w16 = (rng.standard_normal((16, 256)) * 0.05).astype(np.float16)
    a = ingest.quantize_int4(w16, 128)
    b = ingest.quantize_int4(w16.astype(np.float32), 128)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    bits = (rng.integers(0, 1 << 15, (16, 256)) & 0x3FFF | 0x3C00).astype(np.uint16)
    f32 = (bits.astype(np.uint32) << 16).view(np.float32)
    a = ingest.quantize_int4(bits, 128, bf16=True)
    b = ingest.quantize_int4(f32, 128)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
