"""GPU: MoE decode layers served by the VRAM tier (wisp_tier_moe_decode_layer)
against the CPU oracle's run_moe, over a multi-layer decode loop whose
routing makes experts move between VRAM slots, the scratch ring and
promotions, so results depend on every copy being complete and every slot
holding the right blob when it is read.

Bar: the fp16 parity bar of tests/gpu_util.py per token and layer; copy
accounting exact (every lookup that is not a VRAM hit copies one blob)."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import assert_close, make_expert
from wisp_amd import moe, synth, tier
from wisp_amd.hip import DeviceBuffer, PinnedBuffer, Stream, synchronize, to_device

pytestmark = pytest.mark.gpu


def build(L, E, inter, hidden, gs, zeros, seed):
    size = synth.blob_size(inter, hidden, gs)
    pinned = PinnedBuffer(L * E * size)
    host = []
    for l in range(L):
        for e in range(E):
            b = make_expert(seed + 1000 * l, e, inter, hidden, gs, zeros)
            off = (l * E + e) * size
            pinned.array[off:off + size] = b
            host.append(pinned.array[off:off + size])
    ptrs = [pinned.ptr + i * size for i in range(L * E)]
    layout = moe.layout_from_blob(host[0], has_zeros=zeros)
    return pinned, host, ptrs, size, layout


@pytest.mark.parametrize("zeros,shared", [(False, True), (True, False)])
def test_streaming_layers_match_oracle(zeros, shared):
    print(f"tier stream zeros={zeros} shared={shared}", flush=True)
    L, E, inter, hidden, gs, M, k, steps, slots = 3, 12, 256, 512, 128, 2, 3, 12, 5
    rng = np.random.default_rng(5 + zeros)
    pinned, host, ptrs, size, layout = build(L, E, inter, hidden, gs, zeros, 70)
    t = tier.ExpertTier(L, E, size, ptrs, slots, scratch_slots=M * k + 2)
    sh_blobs = [make_expert(900 + l, 0, inter, hidden, gs, zeros) for l in range(L)] if shared else None
    sh_dev = []
    if shared:
        for b in sh_blobs:
            d = DeviceBuffer(b.nbytes + 16)
            d.upload(b, offset=8)
            sh_dev.append(d)
    st = Stream()
    ws = DeviceBuffer(moe.decode_workspace_bytes(layout, M, k, shared))
    out32, out16 = DeviceBuffer(4 * M * hidden), DeviceBuffer(2 * M * hidden)
    not_hits = 0
    for step in range(steps):
        for l in range(L):
            idx = synth.zipf_topk(rng, M, E, k, s=1.1)
            if step == 3 and l == 1:
                idx[1, 2] = -1                           # a skipped slot
            w = synth.route_weights(rng, M, k)
            x = synth.make_x(rng, M, hidden)
            dx = to_device(x)
            before = t.stats()
            t.moe_decode_layer(l, sh_dev[l].ptr + 8 if shared else 0, layout, dx.ptr, M, idx, w, ws,
                               out32.ptr, out16.ptr, st.handle)
            st.synchronize()
            after = t.stats()
            not_hits += (after["lookups"] - before["lookups"]) - (after["vram_hits"] - before["vram_hits"])
            g32 = out32.download(np.float32, (M, hidden))
            g16 = out16.download(np.float16, (M, hidden)).astype(np.float32)
            blobs = host[l * E:(l + 1) * E]
            for v in range(M):
                want = O.moe_combine(blobs, sh_blobs[l] if shared else None, x[v].astype(np.float32),
                                     idx[v], w[v])
                assert_close(g32[v], want, f"step {step} layer {l} token {v} fp32")
                assert_close(g16[v], want, f"step {step} layer {l} token {v} fp16")
    s = t.stats()
    assert s["lookups"] == s["vram_hits"] + s["ram_hits"] + s["first_touch"]
    assert s["h2d_bytes"] == not_hits * size
    assert s["promotions"] > 0 and s["evictions"] > 0 and s["vram_hits"] > 0, s
    t.close()
    synchronize()


def test_rejects_more_experts_than_scratch_slots():
    L, E, inter, hidden, gs = 1, 8, 256, 512, 128
    pinned, host, ptrs, size, layout = build(L, E, inter, hidden, gs, False, 3)
    t = tier.ExpertTier(L, E, size, ptrs, 2, scratch_slots=3)
    with pytest.raises(Exception):
        t.fetch_layer(0, [0, 1, 2, 3])
    paths = t.fetch_layer(0, [0, 1, 2])
    assert paths.tolist() == [tier.COLD_VRAM, tier.COLD_VRAM, tier.COLD_SCRATCH]
    t.close()
    synchronize()
