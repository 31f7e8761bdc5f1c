"""CPU checks of the C-ABI library: it loads, exports every function that
include/wisp_amd.h declares, and its host-only helpers behave. No GPU calls."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from wisp_amd import _lib, synth
from wisp_amd.moe import layout_from_blob

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:[A-Za-z_][\w\s\*]*?)\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M):
            name = m.group(1)
            if name not in {"if", "for", "while", "return", "sizeof"}:
                names.add(name)
    return sorted(names)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = declared_functions()
    assert "wisp_gpu_moe_decode_int4" in declared and "launch_dequant_expert" in declared
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = [n for n in declared if n not in exported]
    assert not missing, missing
    for n in declared:
        assert hasattr(lib, n)
    # every declared function also has a ctypes signature
    assert set(declared) <= set(_lib.signatures())


def test_layout_from_blob_matches_oracle_parser():
    rng = np.random.default_rng(0)
    blob = synth.make_blob(rng, 256, 512, 128)
    L = layout_from_blob(blob)
    m = O.parse_blob(blob)
    assert list(L.packed_off) == list(m.packed_off)
    assert list(L.scales_off) == list(m.scales_off)
    assert list(L.zeros_off) == list(m.zeros_off)
    assert list(L.rows) == list(m.rows) and list(L.cols) == list(m.cols)
    assert L.group_size == 128 and L.total_bytes == blob.nbytes
    lib = _lib.lib()
    bad = blob.copy(); bad[4] = 2
    assert lib.wisp_expert_layout_from_blob(bad.ctypes.data, bad.nbytes, ctypes.byref(L)) == -2
    assert lib.wisp_expert_layout_from_blob(blob.ctypes.data, 64, ctypes.byref(L)) == -1


@pytest.mark.parametrize("inter,hidden,gs,ok", [
    (256, 512, 128, True), (2048, 7168, 128, True), (14336, 4096, 128, True),
    (256, 512, 64, True), (256, 512, 32, True), (256, 512, 256, True),
    (256, 512, 16, False), (192, 512, 64, False), (256, 448, 64, False),
])
def test_layout_check(inter, hidden, gs, ok):
    rng = np.random.default_rng(1)
    hdr = np.zeros(synth.HEADER_BYTES, np.uint8)
    synth.write_header(hdr, 0, 0, inter, hidden, gs)
    full = np.zeros(synth.blob_size(inter, hidden, gs), np.uint8)
    full[:120] = hdr
    L = layout_from_blob(full)
    rc = _lib.lib().wisp_expert_layout_check(ctypes.byref(L))
    assert (rc == 0) == ok


def test_decode_workspace_bytes():
    rng = np.random.default_rng(2)
    blob = synth.make_blob(rng, 256, 512, 128)
    L = layout_from_blob(blob)
    lib = _lib.lib()
    a = lib.wisp_moe_decode_workspace_bytes(ctypes.byref(L), 1, 8, 1)
    b = lib.wisp_moe_decode_workspace_bytes(ctypes.byref(L), 4, 8, 1)
    assert 0 < a < b
    assert lib.wisp_moe_decode_workspace_bytes(ctypes.byref(L), 5, 8, 1) == 0
    assert lib.wisp_moe_decode_workspace_bytes(ctypes.byref(L), 1, 65, 1) == 0


def test_host_side_validation_rejects_without_gpu_calls():
    """Argument checks return hipErrorInvalidValue (1) before any HIP call."""
    lib = _lib.lib()
    fake = 0x1000
    assert lib.launch_dequant_expert(fake, fake, fake, fake, 0, 128, None) == 1
    assert lib.launch_dequant_expert(fake, fake, fake, fake, 128, 0, None) == 1
    rng = np.random.default_rng(3)
    L = layout_from_blob(synth.make_blob(rng, 256, 512, 128))
    ws = lib.wisp_moe_decode_workspace_bytes(ctypes.byref(L), 1, 2, 0)
    args = lambda M, wsb: (fake, None, ctypes.byref(L), fake, 0, M, fake, fake, 2, 8, fake, wsb, 0,
                           fake, None, None)
    assert lib.wisp_gpu_moe_decode_int4(*args(0, ws)) == 1
    assert lib.wisp_gpu_moe_decode_int4(*args(5, ws)) == 1
    assert lib.wisp_gpu_moe_decode_int4(*args(1, ws - 1)) == 1
    # more experts than the prep workgroup's LDS table holds (1024)
    big = (fake, None, ctypes.byref(L), fake, 0, 1, fake, fake, 2, 1025, fake, 1 << 30, 0, fake,
           None, None)
    assert lib.wisp_gpu_moe_decode_int4(*big) == 1
    assert lib.wisp_gpu_moe_layer_decode_int4(fake, None, 0, fake, fake, fake, fake, None,
                                              ctypes.byref(L), fake, 0, 1, 2, 1025, fake, 1 << 30,
                                              0, fake, None, None) == 1
    err = ctypes.c_int(0)
    ptrs = (ctypes.c_void_p * 1025)(*([fake] * 1025))
    assert lib.wisp_tier_create(1, 1025, 4096, ptrs, 4, 10, 3, ctypes.byref(err)) is None
    assert err.value == 1
    L.group_size = 48
    assert lib.wisp_gpu_moe_decode_int4(*args(1, 1 << 30)) == 1
    assert lib.wisp_gpu_moe_route(fake, None, fake, 1, 512, 2048, 8, 0, fake, fake, fake, None) == 1
    assert lib.wisp_gpu_moe_route(fake, None, fake, 1, 512, 256, 8, 7, fake, fake, fake, None) == 1
    assert lib.wisp_gpu_expert_offsets(fake, 1, 8, 5000, fake, fake, fake, fake, None) == 1
    assert lib.wisp_gpu_topk_from_logits(fake, None, 1, 256, 65, 0, fake, fake, fake, None) == 1


def test_header_and_reference_declarations_compile_as_c11():
    """include/wisp_amd.h compiles as C11 with -Werror, and so does the test
    caller that repeats the reference's launcher declarations
    (csrc/core/wisp_engine.h:496-559) with the CUDA type names mapped to HIP:
    C rejects an incompatible repeated declaration."""
    inc = ["-I" + str(ROOT / "include"), "-I/opt/rocm/include", "-D__HIP_PLATFORM_AMD__"]
    flags = ["-std=c11", "-Wall", "-Wextra", "-Werror", "-fsyntax-only"]
    src = ROOT / "tests" / "c_abi" / "engine_call_shape.c"
    r = subprocess.run(["gcc", *flags, *inc, str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    # a changed argument type must be caught
    bad = src.read_text().replace("int rows, int cols, cudaStream_t s);",
                                  "long rows, int cols, cudaStream_t s);", 1)
    r = subprocess.run(["gcc", *flags, *inc, "-x", "c", "-"], input=bad, capture_output=True,
                       text=True)
    assert r.returncode != 0 and "conflicting types" in r.stderr
