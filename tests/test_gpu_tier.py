"""GPU: MoE decode layers served by the VRAM tier (wisp_tier_moe_decode_layer)
against the CPU oracle's run_moe, over a multi-layer decode loop whose
routing makes experts move between VRAM slots, the scratch ring and
promotions, so results depend on every copy being complete and every slot
holding the right blob when it is read.

Bar: the fp16 parity bar of tests/gpu_util.py per token and layer; copy
accounting exact (every lookup that is not a VRAM hit copies one blob)."""
import os

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


@pytest.mark.parametrize("zeros", [False, True])
def test_ssd_tier_streaming_matches_oracle(tmp_path, zeros):
    """Three tiers: expert files on disk (the SSD tier), a RAM tier of 14
    pinned slots, 5 VRAM slots; the routing makes experts drop out of RAM,
    come back from their files, get promoted and evicted (copied back to
    RAM). Every token and layer against the oracle; the executor's paths
    against the policy alone on the same ids; exact byte accounting."""
    print(f"ssd tier zeros={zeros}", flush=True)
    L, E, inter, hidden, gs, M, k, steps, slots, n_ram = 3, 12, 256, 512, 128, 2, 3, 16, 5, 14
    rng = np.random.default_rng(40 + zeros)
    os.makedirs(tmp_path / "experts")
    blobs = {}
    for l in range(L):
        for e in range(E):
            b = make_expert(seed=500 + 1000 * l, e=e, inter=inter, hidden=hidden, gs=gs,
                            zeros=zeros)
            blobs[(l, e)] = b
            b.tofile(tmp_path / "experts" / f"L{l:03d}_E{e:05d}.bin")
    size = synth.blob_size(inter, hidden, gs)
    layout = moe.layout_from_blob(blobs[(0, 0)], has_zeros=zeros)
    t = tier.ExpertTier(L, E, size, None, slots, scratch_slots=M * k + 2,
                        model_path=str(tmp_path), n_ram_slots=n_ram)
    pol = tier.Policy(L, E, slots, M * k + 2, n_ram_slots=n_ram)
    st = Stream()
    ws = DeviceBuffer(moe.decode_workspace_bytes(layout, M, k, False))
    out32 = DeviceBuffer(4 * M * hidden)
    for step in range(steps):
        for l in range(L):
            idx = synth.zipf_topk(rng, M, E, k, s=1.1)
            w = synth.route_weights(rng, M, k)
            x = synth.make_x(rng, M, hidden)
            dx = to_device(x)
            uniq = list(dict.fromkeys(int(e) for e in idx.reshape(-1)))
            pol.begin_layer()
            want_paths = [pol.lookup(l, e)[0] for e in uniq]
            paths = t.fetch_layer(l, uniq, st.handle)
            assert paths.tolist() == want_paths, (step, l)
            t.wait_copies(st.handle)
            di, dw = to_device(idx), to_device(w)
            moe.moe_decode_int4(t.table(l), 0, layout, dx.ptr, M, di.ptr, dw.ptr, k, E, ws,
                                out32=out32.ptr, stream=st.handle)
            t.release_layer(st.handle)
            st.synchronize()
            g32 = out32.download(np.float32, (M, hidden))
            lb = [blobs[(l, e)] for e in range(E)]
            for v in range(M):
                want = O.moe_combine(lb, None, x[v].astype(np.float32), idx[v], w[v])
                assert_close(g32[v], want, f"step {step} layer {l} token {v}")
    s = t.stats()
    ps = pol.stats()
    for key in ("lookups", "vram_hits", "ram_hits", "first_touch", "promotions", "evictions",
                "ram_evictions"):
        assert s[key] == ps[key], key
    assert s["ssd_bytes"] == s["first_touch"] * size
    assert s["h2d_bytes"] == (s["lookups"] - s["vram_hits"]) * size
    assert s["ram_evictions"] > 0 and s["promotions"] > 0 and s["evictions"] > 0, s
    assert s["first_touch"] > len(blobs) // 2
    assert s["d2h_bytes"] > 0 and s["d2h_bytes"] % size == 0   # VRAM victims copied back
    print(f"  stats {s}", flush=True)
    t.close()
    synchronize()


def test_ssd_tier_missing_file_is_an_error(tmp_path):
    os.makedirs(tmp_path / "experts")
    inter, hidden, gs = 256, 512, 128
    b = make_expert(3, 0, inter, hidden, gs)
    b.tofile(tmp_path / "experts" / "L000_E00000.bin")
    t = tier.ExpertTier(1, 4, b.nbytes, None, 2, scratch_slots=3, model_path=str(tmp_path),
                        n_ram_slots=4)
    assert t.fetch_layer(0, [0]).tolist() == [tier.COLD_VRAM]
    with pytest.raises(Exception, match="wisp_tier_fetch_layer"):
        t.fetch_layer(0, [1])
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
