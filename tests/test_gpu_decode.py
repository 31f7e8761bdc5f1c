"""GPU parity of the fused int4 MoE decode (include/wisp_amd.h section 4)
against the CPU oracle's run_moe semantics (shared expert, then routed
experts in rank order, fp32 math), token by token.

Bar: max |gpu - oracle| / max |oracle| <= 1e-2 and cosine >= 0.9999 for the
fp16 and fp32 outputs (tests/gpu_util.py)."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import assert_close, make_expert
from wisp_amd import moe, synth
from wisp_amd.hip import DeviceBuffer, synchronize, to_device

pytestmark = pytest.mark.gpu


def run_decode(seed, inter, hidden, gs, n_exp, top_k, M, shared, zeros, idx, w,
               x_dtype=moe.DTYPE_F16, accumulate=False, full_oracle=True):
    rng = np.random.default_rng(seed)
    used = sorted({int(e) for e in idx.reshape(-1) if 0 <= e < n_exp})
    arena = moe.ExpertArena(n_exp, inter, hidden, gs,
                            lambda e, out: make_expert(seed, e, inter, hidden, gs, zeros, out),
                            has_zeros=zeros, keep_host=used, only=used or [0])
    sh_blob = make_expert(seed, 10_000, inter, hidden, gs, zeros) if shared else None
    sh_dev = None
    if shared:
        sh_dev = DeviceBuffer(sh_blob.nbytes + 16)
        sh_dev.upload(sh_blob, offset=8)
    x = synth.make_x(rng, M, hidden)
    dx = to_device(x if x_dtype == moe.DTYPE_F16 else x.astype(np.float32))
    di, dw = to_device(idx.astype(np.int32)), to_device(w.astype(np.float32))
    ws = DeviceBuffer(moe.decode_workspace_bytes(arena.layout, M, top_k, shared))
    out32, out16 = DeviceBuffer(4 * M * hidden), DeviceBuffer(2 * M * hidden)
    base = rng.standard_normal((M, hidden)).astype(np.float32) if accumulate else None
    if accumulate:
        out32.upload(base)
    moe.moe_decode_int4(arena.table.ptr, sh_dev.ptr + 8 if shared else 0, arena.layout, dx.ptr,
                        M, di.ptr, dw.ptr, top_k, n_exp, ws, out32.ptr, out16.ptr,
                        accumulate=accumulate, x_dtype=x_dtype)
    synchronize()
    g32 = out32.download(np.float32, (M, hidden))
    g16 = out16.download(np.float16, (M, hidden)).astype(np.float32)
    blobs = [arena.host.get(e, arena.host[used[0]] if used else sh_blob) for e in range(n_exp)]
    for t in range(M):
        want = O.moe_combine(blobs, sh_blob, x[t].astype(np.float32), idx[t], w[t])
        if accumulate:
            want = want + base[t]
        assert_close(g32[t], want, f"token {t} fp32")
        assert_close(g16[t], want, f"token {t} fp16")
    return g32


@pytest.mark.parametrize("gs", [128, 64, 32, 256])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_small_shapes(gs, M):
    print(f"decode small gs={gs} M={M}", flush=True)
    rng = np.random.default_rng(100 + gs + M)
    n_exp, k = 8, 2
    idx = synth.uniform_topk(rng, M, n_exp, k)
    w = synth.route_weights(rng, M, k)
    run_decode(gs * 10 + M, 256, 512, gs, n_exp, k, M, shared=True, zeros=True, idx=idx, w=w)


@pytest.mark.parametrize("shared,zeros", [(False, False), (True, False), (False, True)])
def test_small_variants(shared, zeros):
    print(f"decode variants shared={shared} zeros={zeros}", flush=True)
    rng = np.random.default_rng(7)
    n_exp, k, M = 16, 4, 3
    idx = synth.uniform_topk(rng, M, n_exp, k)
    idx[1, 2] = -1                       # skipped slot
    idx[2, 0] = idx[0, 0]                # expert shared between tokens
    w = synth.route_weights(rng, M, k)
    run_decode(77, 384, 640, 128, n_exp, k, M, shared, zeros, idx, w)


@pytest.mark.parametrize("top_k", [8, 12])
def test_repeated_expert_within_token(top_k):
    """Caller-given slots that name one expert twice in one token (and a
    skipped slot): the unique list adds both weights in slot order, as the
    oracle adds both contributions; top_k 12 takes the unique list's
    general scan (more than 8 slots per token)."""
    print(f"decode repeated expert top_k={top_k}", flush=True)
    rng = np.random.default_rng(40 + top_k)
    n_exp, M = 32, 3
    idx = synth.uniform_topk(rng, M, n_exp, top_k)
    idx[1, 3] = idx[1, 0]                # same expert twice in token 1
    idx[2, 5] = -1                       # skipped slot
    idx[0, 1] = idx[2, 2]                # expert shared between tokens
    w = synth.route_weights(rng, M, top_k)
    run_decode(500 + top_k, 256, 512, 128, n_exp, top_k, M, True, False, idx, w)


def test_fp32_input_and_accumulate():
    rng = np.random.default_rng(8)
    idx = synth.uniform_topk(rng, 2, 8, 2)
    w = synth.route_weights(rng, 2, 2)
    run_decode(88, 256, 512, 128, 8, 2, 2, True, True, idx, w, x_dtype=moe.DTYPE_F32, accumulate=True)


@pytest.mark.parametrize("M", [1, 4])
def test_mixtral_shape(M):
    print(f"decode mixtral M={M}", flush=True)
    s = synth.MIXTRAL
    rng = np.random.default_rng(1000 + M)
    idx = synth.uniform_topk(rng, M, s.n_experts, s.top_k)
    w = synth.route_weights(rng, M, s.top_k)
    run_decode(2000 + M, s.inter, s.hidden, s.group_size, s.n_experts, s.top_k, M, False, False,
               idx, w)


@pytest.mark.parametrize("M", [1, 2, 4])
def test_dsv3_shape(M):
    print(f"decode dsv3 M={M}", flush=True)
    s = synth.DSV3
    rng = np.random.default_rng(3000 + M)
    idx = synth.uniform_topk(rng, M, s.n_experts, s.top_k)
    w = synth.route_weights(rng, M, s.top_k)
    run_decode(4000 + M, s.inter, s.hidden, s.group_size, s.n_experts, s.top_k, M, True, False,
               idx, w)


@pytest.mark.parametrize("hidden,gs,zeros,M", [(7168, 128, False, 1), (7168, 32, True, 1),
                                                (5120, 64, False, 1), (4608, 128, True, 1),
                                                (12288, 256, False, 1), (7168, 128, True, 2),
                                                (7168, 64, False, 3), (7168, 128, False, 4),
                                                (12288, 128, True, 4), (5120, 128, False, 2)])
def test_split_gate_up(hidden, gs, zeros, M):
    """More than 32 hidden blocks: each gate/up row tile's K axis is split
    over several workgroups (7 blocks per wave at 56 blocks, otherwise 8 with
    idle waves in the last split), for one token in the one-launch kernel and
    for 2-4 tokens in the separate gate/up launch; two calls in a row on one
    workspace give identical results."""
    print(f"decode split gate/up hidden={hidden} gs={gs} zeros={zeros} M={M}", flush=True)
    rng = np.random.default_rng(hidden + gs + M)
    n_exp, k = 16, 4
    idx = synth.uniform_topk(rng, M, n_exp, k)
    w = synth.route_weights(rng, M, k)
    a = run_decode(hidden + 3 * gs + M, 256, hidden, gs, n_exp, k, M, True, zeros, idx, w)
    b = run_decode(hidden + 3 * gs + M, 256, hidden, gs, n_exp, k, M, True, zeros, idx, w)
    np.testing.assert_array_equal(a, b)


def test_invalid_arguments_are_rejected():
    rng = np.random.default_rng(9)
    blob = synth.make_blob(rng, 256, 512, 128)
    L = moe.layout_from_blob(blob)
    ws = DeviceBuffer(moe.decode_workspace_bytes(L, 1, 2, False))
    d = DeviceBuffer(1 << 16)
    with pytest.raises(Exception):
        moe.moe_decode_int4(d.ptr, 0, L, d.ptr, 5, d.ptr, d.ptr, 2, 8, ws, d.ptr)
    small = DeviceBuffer(64)
    with pytest.raises(Exception):
        moe.moe_decode_int4(d.ptr, 0, L, d.ptr, 1, d.ptr, d.ptr, 2, 8, small, d.ptr)
    # expert count and top-k past the documented ranges are rejected before any launch
    big = DeviceBuffer(moe.decode_workspace_bytes(L, 1, 64, False))
    for k, n_exp in ((65, 128), (0, 8), (2, 1025), (2, 0)):
        with pytest.raises(Exception):
            moe.moe_decode_int4(d.ptr, 0, L, d.ptr, 1, d.ptr, d.ptr, k, n_exp, big, d.ptr)
