"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each oracle function is checked against at least one of: the reference's
own known-answer tests, the reference's scalar C compiled from its sources
(oracle/_ref, present when the reference tree was available at build time),
the committed golden fixtures, or a closed form / float64 brute force that
a plausible mistake (swapped nibbles, dropped zero term, wrong group index,
wrong tie rule) would fail.
"""
import struct

import numpy as np
import pytest

from oracle import oracle as O
from wisp_amd import synth

REF = O.LazyRef()   # loaded by the first test that uses it, not at import
needs_ref = pytest.mark.skipif(not O.ref_built(), reason="reference tree not built into oracle/_ref")


# --------------------------------------------------------------------------
# fp16 conversions
# --------------------------------------------------------------------------

def test_half_to_float_exhaustive_vs_ieee():
    o = O.orc()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([o.orc_half_to_float(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@needs_ref
def test_half_to_float_matches_reference_helper():
    o = O.orc()
    for b in range(0, 65536, 7):
        a, r = o.orc_half_to_float(b), REF.ref_half_to_float(b)
        assert (np.isnan(a) and np.isnan(r)) or np.float32(a).view(np.uint32) == np.float32(r).view(np.uint32)


def test_float_to_half_rne_vs_numpy():
    o = O.orc()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8,
                  1e-9, -1e-9, np.inf, -np.inf, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11], np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):   # values past 65519.99 round to inf on purpose
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([o.orc_float_to_half(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)


@needs_ref
def test_float_to_half_trunc_matches_reference_helper():
    o = O.orc()
    rng = np.random.default_rng(1)
    vals = rng.standard_normal(5000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 5, 5000)
    for v in vals:
        assert o.orc_float_to_half_trunc(float(v)) == REF.ref_float_to_half(float(v))


# --------------------------------------------------------------------------
# int4 format
# --------------------------------------------------------------------------

def test_constant_group_packs_to_0x88():
    """Known answer of tests/test_adapters.py:262-267: a constant group
    quantises to nibble 8 everywhere, i.e. byte 0x88, and dequantises to the
    zero point exactly."""
    nib = np.full(64, 8, np.uint8)
    packed = np.empty(32, np.uint8)
    O.orc().orc_pack_int4(O._p(nib), 64, O._p(packed))
    assert packed[0] == 0x88 and np.all(packed == 0x88)
    one = np.array([np.float16(1.0).view(np.uint16)], np.uint16)
    zero_scale = np.array([0], np.uint16)
    out = O.dequant_f32(packed, zero_scale, one, 64, 64)
    assert np.all(out == 1.0)


def test_unpack_low_nibble_is_even_index():
    packed = np.array([0x21, 0x43, 0xF0], np.uint8)
    nib = np.empty(6, np.uint8)
    O.orc().orc_unpack_int4(O._p(packed), 6, O._p(nib))
    assert nib.tolist() == [1, 2, 3, 4, 0, 15]
    back = np.empty(3, np.uint8)
    O.orc().orc_pack_int4(O._p(nib), 6, O._p(back))
    assert np.array_equal(back, packed)
    # odd tail pads the final high nibble with 0 (quantizer.py:75-79)
    odd = np.empty(2, np.uint8)
    O.orc().orc_pack_int4(O._p(nib[:3]), 3, O._p(odd))
    assert odd.tolist() == [0x21, 0x03]


def _closed_form_dequant(packed, scales, zeros, n, gs):
    nib = np.empty(2 * len(packed), np.int32)
    nib[0::2] = packed & 0x0F
    nib[1::2] = packed >> 4
    g = np.arange(n) // gs
    s = scales.view(np.float16).astype(np.float32)[g]
    z = zeros.view(np.float16).astype(np.float32)[g]
    return (nib[:n].astype(np.float32) - np.float32(8)) * s + z


@pytest.mark.parametrize("gs", [16, 64, 128, 37])
def test_dequant_matches_closed_form(gs):
    rng = np.random.default_rng(gs)
    n = 4096 + (gs == 37) * 3
    packed = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
    ng = (n + gs - 1) // gs
    scales = (np.abs(rng.standard_normal(ng)) * 0.01).astype(np.float16).view(np.uint16)
    zeros = (rng.standard_normal(ng) * 0.01).astype(np.float16).view(np.uint16)
    want = _closed_form_dequant(packed, scales, zeros, n, gs)
    f32 = O.dequant_f32(packed, scales, zeros, n, gs)
    assert np.array_equal(f32.view(np.uint32), want.view(np.uint32))
    f16 = O.dequant_fp16(packed, scales, zeros, n, gs)
    assert np.array_equal(f16, want.astype(np.float16).view(np.uint16))


def test_dequant_golden_fixture():
    g = np.load(synth_golden("dequant_g64.npz"))
    f16 = O.dequant_fp16(g["packed"], g["scales"], g["zeros"], int(g["n"]), int(g["gs"]))
    assert np.array_equal(f16, g["out_f16"])


@needs_ref
def test_dequant_matches_reference_probe(tmp_path):
    """The reference's own byte-layout cross-check (tests/test_adapters.py:
    311-345, csrc/core/wisp_engine.c:311-349), run on a blob written here."""
    rng = np.random.default_rng(7)
    inter, hidden, gs = 16, 32, 16
    blob = synth.make_blob(rng, inter, hidden, gs, layer=5, expert=123, zeros=True)
    path = tmp_path / "L005_E00123.bin"
    path.write_bytes(blob.tobytes())
    for mat, (p, s, z, r, c) in enumerate(synth.blob_views(blob, inter, hidden, gs)):
        out = np.empty(r * c, np.float32)
        assert REF.ref_debug_probe(str(path).encode(), mat, r * c, O._p(out)) == 0
        mine = O.dequant_f32(p, s, z, r * c, gs)
        assert np.array_equal(out.view(np.uint32), mine.view(np.uint32))


# --------------------------------------------------------------------------
# blob layout
# --------------------------------------------------------------------------

def test_blob_layout_constants():
    """tests/test_adapters.py:281-308: 120-byte header, sections tile the file."""
    rng = np.random.default_rng(1)
    inter, hidden, gs = 16, 32, 16
    blob = synth.make_blob(rng, inter, hidden, gs, layer=3, expert=42)
    assert synth.HEADER_BYTES == 120
    magic, ver, layer, expert, group, nmats = struct.unpack_from("<6I", blob)
    assert (magic, ver, layer, expert, group, nmats) == (0x57455850, 1, 3, 42, gs, 3)
    m = O.parse_blob(blob)
    assert m.total_bytes == blob.nbytes == O.orc().orc_blob_size(inter, hidden, gs)
    assert list(m.rows) == [16, 16, 32] and list(m.cols) == [32, 32, 16]
    assert m.packed_off[0] == 120


def test_blob_parse_rejects_bad_headers():
    rng = np.random.default_rng(2)
    blob = synth.make_blob(rng, 16, 32, 16)
    o = O.orc()
    m = O.BlobMeta()
    assert o.orc_blob_parse(O._p(blob), 100, O.ctypes.byref(m)) == -1
    bad = blob.copy(); bad[0] ^= 1
    assert o.orc_blob_parse(O._p(bad), bad.nbytes, O.ctypes.byref(m)) == -2
    assert o.orc_blob_parse(O._p(blob), blob.nbytes - 1, O.ctypes.byref(m)) == -3


@needs_ref
def test_blob_parse_matches_reference_parser():
    rng = np.random.default_rng(3)
    blob = synth.make_blob(rng, 256, 128, 64)
    out = np.zeros(14, np.uint64)
    assert REF.ref_parse_header(O._p(blob), blob.nbytes, O._p(out)) == 0
    m = O.parse_blob(blob)
    assert list(out[0:3]) == list(m.rows) and list(out[3:6]) == list(m.cols)
    assert list(out[6:9]) == list(m.packed_off) and list(out[9:12]) == list(m.scales_off)
    assert out[12] == m.group_size and out[13] == m.total_bytes


# --------------------------------------------------------------------------
# expert math
# --------------------------------------------------------------------------

def _mat(rng, rows, cols, gs, zeros=True):
    n = rows * cols
    packed = rng.integers(0, 256, n // 2, dtype=np.uint8)
    scales = (np.abs(rng.standard_normal(n // gs)) * 0.01).astype(np.float16).view(np.uint16)
    z = (rng.standard_normal(n // gs) * 0.01) if zeros else np.zeros(n // gs)
    return packed, scales, z.astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("rows,cols,gs", [(64, 256, 64), (32, 512, 128), (16, 96, 32)])
def test_gemv_int4_vs_float64_brute_force(rows, cols, gs):
    rng = np.random.default_rng(rows + cols)
    packed, scales, zeros = _mat(rng, rows, cols, gs)
    x = rng.standard_normal(cols).astype(np.float32)
    W = _closed_form_dequant(packed, scales, zeros, rows * cols, gs).astype(np.float64).reshape(rows, cols)
    want = W @ x.astype(np.float64)
    got = O.gemv_int4(packed, scales, zeros, x, rows, cols, gs)
    bound = 64 * np.finfo(np.float32).eps * (np.abs(W) @ np.abs(x))
    assert np.all(np.abs(got - want) <= bound)
    f64 = O.gemv_int4_f64(packed, scales, zeros, x, rows, cols, gs)
    assert np.allclose(f64, want, rtol=1e-12, atol=1e-12)
    # a plausible mistake fails: dropping the zero term
    nozero = O.gemv_int4(packed, scales, np.zeros_like(zeros), x, rows, cols, gs)
    assert np.max(np.abs(nozero - want)) > 1e3 * np.max(bound)


@needs_ref
@pytest.mark.parametrize("rows,cols,gs", [(128, 512, 64), (64, 1024, 128)])
def test_gemv_int4_matches_reference_scalar_c(rows, cols, gs):
    rng = np.random.default_rng(11)
    packed, scales, zeros = _mat(rng, rows, cols, gs)
    x = rng.standard_normal(cols).astype(np.float32)
    got = O.gemv_int4(packed, scales, zeros, x, rows, cols, gs)
    ref = np.empty(rows, np.float32)
    REF.ref_gemv_int4(O._p(packed), O._p(scales), O._p(zeros), O._p(x), O._p(ref), rows, cols, gs)
    # same fp32 sequence up to fused multiply-add contraction in the build
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_fast_baseline_matches_scalar_oracle():
    rng = np.random.default_rng(12)
    rows, cols, gs = 256, 2048, 128
    packed, scales, zeros = _mat(rng, rows, cols, gs)
    x = rng.standard_normal(cols).astype(np.float32)
    a = O.gemv_int4(packed, scales, zeros, x, rows, cols, gs)
    b = O.gemv_int4(packed, scales, zeros, x, rows, cols, gs, fast=True)
    assert np.max(np.abs(a - b)) <= 1e-5 * np.max(np.abs(a))


@needs_ref
def test_swiglu_matches_reference():
    rng = np.random.default_rng(4)
    g = rng.standard_normal(1000).astype(np.float32) * 4
    u = rng.standard_normal(1000).astype(np.float32)
    mine = np.empty_like(g)
    O.orc().orc_swiglu(O._p(g), O._p(u), O._p(mine), 1000)
    ref = np.empty_like(g)
    REF.ref_swiglu(O._p(g), O._p(u), O._p(ref), 1000)
    assert np.array_equal(mine, ref)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(mine, want, rtol=1e-6, atol=1e-7)


@needs_ref
@pytest.mark.parametrize("zeros", [False, True])
def test_expert_ffn_matches_reference(zeros):
    rng = np.random.default_rng(5)
    inter, hidden, gs = 256, 512, 128
    blob = synth.make_blob(rng, inter, hidden, gs, zeros=zeros)
    x = rng.standard_normal(hidden).astype(np.float16).astype(np.float32)
    acc0 = rng.standard_normal(hidden).astype(np.float32)
    mine = O.expert_ffn(blob, x, acc0.copy(), 0.37)
    ref = acc0.copy()
    assert REF.ref_expert_ffn(O._p(blob), blob.nbytes, O._p(x), O._p(ref), np.float32(0.37)) == 0
    assert np.max(np.abs(mine - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_expert_ffn_vs_float64_composition():
    rng = np.random.default_rng(6)
    inter, hidden, gs = 128, 256, 64
    blob = synth.make_blob(rng, inter, hidden, gs, zeros=True)
    x = rng.standard_normal(hidden).astype(np.float32)
    mats = [(_closed_form_dequant(p, s, z, r * c, gs).astype(np.float64).reshape(r, c))
            for p, s, z, r, c in synth.blob_views(blob, inter, hidden, gs)]
    g, u = mats[0] @ x, mats[1] @ x
    h = g / (1 + np.exp(-g)) * u
    want = 0.5 * (mats[2] @ h)
    got = O.expert_ffn(blob, x, None, 0.5)
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want))


# --------------------------------------------------------------------------
# routing
# --------------------------------------------------------------------------

def _brute_topk(scores, k):
    order = sorted(range(len(scores)), key=lambda e: (-scores[e], e))
    return [e for e in order if scores[e] > -1.0][:k]


def test_topk_select_ties_to_lowest_index():
    s = np.array([0.1, 0.5, 0.5, 0.2, 0.5, -2.0], np.float32)
    idx, val = O.topk_select(s, 4)
    assert idx.tolist() == [1, 2, 4, 3]
    assert idx.tolist() == _brute_topk(s, 4)
    rng = np.random.default_rng(8)
    for _ in range(50):
        s = rng.integers(0, 6, 40).astype(np.float32) / 5
        idx, _ = O.topk_select(s, 7)
        assert idx.tolist() == _brute_topk(s, 7)
    # scores <= -1 are never picked (bestv starts at -1)
    idx, _ = O.topk_select(np.array([-1.0, -3.0], np.float32), 2)
    assert idx.tolist() == [-1, -1]


@needs_ref
def test_softmax_router_matches_reference():
    rng = np.random.default_rng(9)
    for n_exp, hidden, k in [(8, 256, 2), (64, 512, 8)]:
        W = synth.make_router(rng, n_exp, hidden)
        bias = (rng.standard_normal(n_exp) * 0.1).astype(np.float16).view(np.uint16)
        x = rng.standard_normal(hidden).astype(np.float32)
        for b in (None, bias):
            idx, w, _ = O.router_topk(W.view(np.uint16), b, x, k)
            ridx = np.empty(k, np.int32); rw = np.empty(k, np.float32); lg = np.empty(n_exp, np.float32)
            REF.ref_router_topk(O._p(W), None if b is None else O._p(b), O._p(x), O._p(lg), n_exp,
                                hidden, k, O._p(ridx), O._p(rw))
            assert idx.tolist() == ridx.tolist()
            assert np.allclose(w, rw, rtol=1e-5)


def test_softmax_router_closed_form():
    rng = np.random.default_rng(10)
    W = synth.make_router(rng, 16, 128)
    x = rng.standard_normal(128).astype(np.float32)
    idx, w, _ = O.router_topk(W.view(np.uint16), None, x, 4)
    l = W.astype(np.float64) @ x
    top = np.argsort(-l, kind="stable")[:4]
    assert idx.tolist() == top.tolist()
    p = np.exp(l[top] - l.max())
    assert np.allclose(w, p / p.sum(), rtol=1e-5)


def test_sigmoid_router_closed_form():
    rng = np.random.default_rng(11)
    W = synth.make_router(rng, 64, 256, std=0.1)
    x = rng.standard_normal(256).astype(np.float32)
    idx, w, _ = O.router_topk(W.view(np.uint16), None, x, 8, kind="sigmoid")
    l = W.astype(np.float64) @ x
    top = np.argsort(-l, kind="stable")[:8]
    assert idx.tolist() == top.tolist()
    s = 1 / (1 + np.exp(-l[top]))
    assert np.allclose(w, s / s.sum(), rtol=1e-5)
    # bias affects selection only
    bias = np.zeros(64, np.float16); bias[top[-1]] = -5.0
    idx2, w2, _ = O.router_topk(W.view(np.uint16), bias.view(np.uint16), x, 8, kind="sigmoid")
    assert top[-1] not in idx2.tolist()
    s2 = 1 / (1 + np.exp(-l[idx2]))
    assert np.allclose(w2, s2 / s2.sum(), rtol=1e-5)


def test_expert_offsets_closed_form():
    rng = np.random.default_rng(12)
    for n_tok, k, n_exp in [(1, 8, 256), (4, 2, 8), (300, 8, 64)]:
        t = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
        if n_tok > 2:
            t[1, 0] = -1          # skipped pair
        counts, offsets, order = O.expert_offsets(t, n_exp)
        flat = t.reshape(-1)
        valid = flat >= 0
        assert np.array_equal(counts, np.bincount(flat[valid], minlength=n_exp))
        assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts)
        want = np.argsort(np.where(valid, flat, n_exp), kind="stable")[: valid.sum()]
        assert np.array_equal(order[: valid.sum()], want)


def test_moe_combine_is_shared_then_rank_order():
    rng = np.random.default_rng(13)
    inter, hidden, gs = 128, 128, 64
    blobs = [synth.make_blob(rng, inter, hidden, gs, expert=e) for e in range(4)]
    shared = synth.make_blob(rng, inter, hidden, gs, expert=99)
    x = rng.standard_normal(hidden).astype(np.float32)
    idx = np.array([2, 0], np.int32)
    w = np.array([0.7, 0.3], np.float32)
    got = O.moe_combine(blobs, shared, x, idx, w)
    acc = O.expert_ffn(shared, x, None, 1.0)
    acc = O.expert_ffn(blobs[2], x, acc, 0.7)
    acc = O.expert_ffn(blobs[0], x, acc, 0.3)
    assert np.array_equal(got, acc)


def test_fast_combine_matches_scalar_combine():
    """moe_combine(fast=True), which the config-scale GPU tests use, against
    the scalar restatement: same order (shared, then rank order), vectorised
    dot products."""
    rng = np.random.default_rng(31)
    inter, hidden, gs = 256, 1024, 128
    blobs = [synth.make_blob(rng, inter, hidden, gs, expert=e) for e in range(6)]
    shared = synth.make_blob(rng, inter, hidden, gs, expert=99)
    x = rng.standard_normal(hidden).astype(np.float32)
    idx = np.array([4, -1, 1], np.int32)
    w = np.array([0.5, 0.2, 0.3], np.float32)
    a = O.moe_combine(blobs, shared, x, idx, w)
    b = O.moe_combine(blobs, shared, x, idx, w, fast=True)
    assert np.max(np.abs(a - b)) <= 1e-5 * np.max(np.abs(a))
    c = O.moe_combine(blobs, shared, x, np.array([4, 1], np.int32), np.array([0.5, 0.3], np.float32))
    assert np.array_equal(a, c)   # a skipped slot contributes nothing


def test_fill_random_bytes_is_deterministic_and_uniform():
    """The synthetic-byte generator of the config-scale tests: a pure
    function of (seed, position), so a longer fill extends a shorter one,
    seeds differ, and byte values are close to uniform."""
    a = O.random_bytes(1 << 20, 7)
    assert np.array_equal(a, O.random_bytes(1 << 20, 7))
    assert np.array_equal(a[:1001], O.random_bytes(1001, 7))
    assert not np.array_equal(a, O.random_bytes(1 << 20, 8))
    h = np.bincount(a, minlength=256)
    assert h.min() > 0.9 * (1 << 12) and h.max() < 1.1 * (1 << 12)


@needs_ref
def test_reference_lru_selftest():
    assert REF.ref_selftest_lru() == 1


def synth_golden(name):
    import os
    return os.path.join(os.path.dirname(__file__), "golden", name)


# --------------------------------------------------------------------------
# oracle vs the committed fixtures (expected outputs produced by the
# reference's own compiled C; these run where the reference tree is absent)
# --------------------------------------------------------------------------

def test_oracle_vs_golden_gemv():
    g = np.load(synth_golden("gemv_int4.npz"))
    y = O.gemv_int4(g["packed"], g["scales"], g["zeros"], g["x"], int(g["rows"]), int(g["cols"]), int(g["gs"]))
    assert np.max(np.abs(y - g["y"])) <= 1e-5 * np.max(np.abs(g["y"]))


def test_oracle_vs_golden_expert_ffn():
    g = np.load(synth_golden("expert_ffn.npz"))
    out = O.expert_ffn(g["blob"], g["x"], g["acc"].copy(), float(g["w"]))
    assert np.max(np.abs(out - g["out"])) <= 1e-5 * np.max(np.abs(g["out"]))


def test_oracle_vs_golden_router():
    g = np.load(synth_golden("router_softmax.npz"))
    idx, w, probs = O.router_topk(g["W"], g["bias"], g["x"], int(g["k"]))
    assert idx.tolist() == g["idx"].tolist()
    assert np.allclose(w, g["w"], rtol=1e-5)
    assert np.allclose(probs, g["probs"], rtol=1e-5, atol=1e-9)


# --------------------------------------------------------------------------
# the decode step's neighbouring ops (RMSNorm, residual, transposed GEMV)
# --------------------------------------------------------------------------

def test_layer_ops_vs_golden():
    """Fixture written by the reference's scalar C (tests/golden/make_golden.py)."""
    g = np.load(synth_golden("layer_ops.npz"))
    assert np.array_equal(O.rmsnorm(g["x"], g["w"], float(g["eps"])), g["y"])
    # the reference build contracts a * b + acc into an FMA; the oracle does
    # not (-ffp-contract=off): same sum order, last-bit differences
    yt = O.gemv_t_f16(g["Wt"], g["xt"])
    assert np.max(np.abs(yt - g["yt"])) <= 1e-6 * np.max(np.abs(g["yt"]))
    assert np.array_equal(O.residual_add(g["r0"], g["d"]), g["r1"])


@needs_ref
def test_layer_ops_match_reference_scalar_c():
    rng = np.random.default_rng(41)
    for n in (1, 7, 4096, 7169):
        x = (rng.standard_normal(n) * 2).astype(np.float32)
        w = (1 + 0.2 * rng.standard_normal(n)).astype(np.float16)
        want = np.empty(n, np.float32)
        REF.ref_rmsnorm(O._p(x), O._p(w), O._p(want), n, np.float32(1e-5))
        assert np.array_equal(O.rmsnorm(x, w, 1e-5), want)
    W = (rng.standard_normal((33, 70)) * 0.1).astype(np.float16)
    xt = rng.standard_normal(33).astype(np.float32)
    want = np.empty(70, np.float32)
    REF.ref_gemv_t_f16(O._p(W), O._p(xt), O._p(want), 33, 70)
    assert np.max(np.abs(O.gemv_t_f16(W, xt) - want)) <= 1e-6 * np.max(np.abs(want))


def test_layer_ops_closed_forms():
    """RMSNorm against float64 (scale applied to x, then the fp16 weight;
    a wrong mean or a missing eps fails), and W^T x against the transposed
    product."""
    rng = np.random.default_rng(42)
    n = 1000
    x = rng.standard_normal(n).astype(np.float32)
    w = (1 + 0.3 * rng.standard_normal(n)).astype(np.float16)
    eps = 1e-2
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps) * \
        w.astype(np.float64)
    got = O.rmsnorm(x, w, eps)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))
    z = O.rmsnorm(np.zeros(16, np.float32), np.ones(16, np.float16), 1e-6)
    assert not np.any(z)
    W = rng.standard_normal((40, 24)).astype(np.float16)
    xt = rng.standard_normal(40).astype(np.float32)
    want = W.astype(np.float64).T @ xt.astype(np.float64)
    assert np.max(np.abs(O.gemv_t_f16(W, xt) - want)) <= 1e-5 * np.max(np.abs(want))


def test_valid_topk_checker_accepts_ties_and_rejects_wrong_selections():
    """The near-tie check the GPU routing tests fall back on: it accepts any
    order of tied keys and rejects a selection that misses a clearly larger
    key, repeats an expert, takes a non-selectable one or is out of rank
    order (mistakes planted here, on the CPU)."""
    from tests.gpu_util import assert_valid_topk
    keys = np.array([0.5, 2.0, 2.0 + 1e-9, -np.inf, 1.0, 2.0 - 1e-9, np.nan, 0.1])
    tol = 1e-6
    assert_valid_topk(keys, [2, 1, 5], 3, tol)        # the three tied keys, any order
    assert_valid_topk(keys, [5, 2, 1], 3, tol)
    assert_valid_topk(keys, [2, 1, 5, 4], 4, tol)
    bad = [([2, 1, 4], "misses a larger key"), ([2, 2, 5], "repeats"),
           ([2, 1, 3], "non-selectable"), ([4, 2, 1, 5], "out of rank order"),
           ([2, 1], "too few")]
    for sel, why in bad:
        k = 4 if len(sel) == 4 else 3
        with pytest.raises(AssertionError):
            assert_valid_topk(keys, sel, k, tol)
            print("accepted", why)
    # fewer selectable keys than k: all of them, then -1
    few = np.array([np.nan, 3.0, -np.inf, 1.0])
    assert_valid_topk(few, [1, 3, -1, -1], 4, tol)
    with pytest.raises(AssertionError):
        assert_valid_topk(few, [1, -1, -1, -1], 4, tol)
