"""VRAM-tier policy (include/wisp_amd.h section 6) on the host, no GPU.

Pinned against the reference's own tier code: oracle/_ref compiles
csrc/core/wisp_engine.c (wisp_expert_fetch, :1138-1296) with its LRU
(lru_cache.c) and VRAM budget (mem_pool.c) on the host, reading expert files
from disk. For the same Zipf routing trace both must take the same path on
every lookup (VRAM hit / RAM hit via scratch / RAM hit promoted / first
touch into VRAM / first touch via scratch) and end with the same counters.
Hand-worked traces pin the rules where the reference tree is absent."""
import os

import numpy as np
import pytest

from oracle import oracle as O
from wisp_amd import synth, tier

REF = O.LazyRef()   # loaded by the first test that uses it, not at import
needs_ref = pytest.mark.skipif(not O.ref_built(), reason="reference tree not built into oracle/_ref")


def zipf_trace(rng, steps, n_layers, n_experts, k):
    return [[synth.zipf_topk(rng, 1, n_experts, k)[0] for _ in range(n_layers)]
            for _ in range(steps)]


@needs_ref
@pytest.mark.parametrize("n_slots,seed", [(6, 1), (10, 2), (20, 3), (0, 4)])
def test_paths_match_reference(tmp_path, n_slots, seed):
    L, E, k, steps = 3, 16, 4, 40
    inter, hidden, gs = 128, 128, 128
    os.makedirs(tmp_path / "experts")
    size = None
    for l in range(L):
        for e in range(E):
            b = synth.make_blob(np.random.default_rng([l, e]), inter, hidden, gs, layer=l, expert=e)
            size = b.nbytes
            b.tofile(tmp_path / "experts" / f"L{l:03d}_E{e:05d}.bin")
    scratch = min(k + 2, 16)
    ref = REF.ref_tier_create(str(tmp_path).encode(), L, k, size, n_slots * size, 1 << 40)
    pol = tier.Policy(L, E, n_slots, scratch)
    trace = zipf_trace(np.random.default_rng(seed), steps, L, E, k)
    seen = {p: 0 for p in range(5)}
    for t, layers in enumerate(trace):
        for l, ids in enumerate(layers):
            pol.begin_layer()
            for e in ids:
                want = REF.ref_tier_fetch(ref, l, int(e))
                got, slot, _ = pol.lookup(l, int(e))
                assert got == want, (t, l, int(e), got, want)
                seen[got] += 1
    counts = (np.zeros(5, np.uint64))
    REF.ref_tier_stats(ref, counts.ctypes.data)
    st = pol.stats()
    assert st["vram_hits"] == counts[0]
    assert st["ram_hits"] == counts[1]
    assert st["first_touch"] == counts[2]
    # every path the policy has was exercised by at least one of the traces
    if n_slots == 10:
        assert all(seen[p] > 0 for p in range(5)), seen


@needs_ref
@pytest.mark.parametrize("n_slots,n_ram,seed", [(6, 12, 5), (10, 8, 6), (4, 24, 7), (0, 10, 8),
                                                (12, 30, 9)])
def test_paths_match_reference_with_bounded_ram(tmp_path, n_slots, n_ram, seed):
    """The three-tier case: the reference's RAM LRU with a byte budget of
    n_ram blobs (entries dropped when full, hit counts lost, VRAM victims
    copied back) against the policy's bounded RAM tier, path by path."""
    L, E, k, steps = 3, 16, 4, 60
    inter, hidden, gs = 128, 128, 128
    os.makedirs(tmp_path / "experts")
    size = None
    for l in range(L):
        for e in range(E):
            b = synth.make_blob(np.random.default_rng([l, e]), inter, hidden, gs, layer=l, expert=e)
            size = b.nbytes
            b.tofile(tmp_path / "experts" / f"L{l:03d}_E{e:05d}.bin")
    scratch = min(k + 2, 16)
    ref = REF.ref_tier_create(str(tmp_path).encode(), L, k, size, n_slots * size, n_ram * size)
    pol = tier.Policy(L, E, n_slots, scratch, n_ram_slots=n_ram)
    trace = zipf_trace(np.random.default_rng(seed), steps, L, E, k)
    seen = {p: 0 for p in range(5)}
    for t, layers in enumerate(trace):
        for l, ids in enumerate(layers):
            pol.begin_layer()
            for e in ids:
                want = REF.ref_tier_fetch(ref, l, int(e))
                got, _, _ = pol.lookup(l, int(e))
                assert got == want, (t, l, int(e), got, want)
                seen[got] += 1
    counts = np.zeros(5, np.uint64)
    REF.ref_tier_stats(ref, counts.ctypes.data)
    st = pol.stats()
    assert (st["vram_hits"], st["ram_hits"], st["first_touch"]) == tuple(int(c) for c in counts[:3])
    if n_ram < L * E:
        assert st["ram_evictions"] > 0
        # more SSD reads than distinct experts: some came back after a RAM eviction
        distinct = len({(l, int(e)) for layers in trace for l, ids in enumerate(layers) for e in ids})
        assert st["first_touch"] > distinct


def test_bounded_ram_drops_hit_counts():
    """An expert dropped from the RAM tier loses its hit count: it comes
    back as an SSD miss and needs three more RAM hits to be promoted."""
    p = tier.Policy(1, 8, 1, 2, n_ram_slots=3)
    order = [0, 0, 1, 2, 3, 0, 0, 0, 0]
    paths = []
    for e in order:
        p.begin_layer()
        paths.append(p.lookup(0, e)[0])
    # 0 takes the one VRAM slot; 1, 2, 3 are SSD misses through scratch, and
    # 3 drops the LRU RAM entry (0, which sits in VRAM); 0 is still a VRAM hit
    assert paths[:5] == [tier.COLD_VRAM, tier.VRAM_HIT, tier.COLD_SCRATCH, tier.COLD_SCRATCH,
                         tier.COLD_SCRATCH]
    assert paths[5:] == [tier.VRAM_HIT] * 4
    st = p.stats()
    assert st["ram_evictions"] == 1 and st["first_touch"] == 4
    q = tier.Policy(1, 8, 0, 2, n_ram_slots=3)
    paths = []
    for e in [5, 5, 6, 7, 4, 5, 5, 5]:
        q.begin_layer()
        paths.append(q.lookup(0, e)[0])
    # 5 earns one RAM hit, is dropped by 4 (LRU after 6, 7 came in), then is an
    # SSD miss again with a fresh count: two RAM hits later it still rides scratch
    assert paths == [tier.COLD_SCRATCH, tier.RAM_SCRATCH, tier.COLD_SCRATCH, tier.COLD_SCRATCH,
                     tier.COLD_SCRATCH, tier.COLD_SCRATCH, tier.RAM_SCRATCH, tier.RAM_SCRATCH]
    with pytest.raises(ValueError):
        tier.Policy(1, 8, 0, 4, n_ram_slots=4)       # must exceed the scratch ring


def test_promotion_on_third_ram_hit_and_lru_eviction():
    # 1 layer, 4 experts, 2 slots, scratch ring of 3. A first touch sets the
    # RAM hit count to 0 (the reference's SSD-miss path); promotion comes on
    # the third RAM hit, i.e. the fourth touch.
    p = tier.Policy(1, 4, 2, 3)
    seq = []
    for e in [0, 1, 2, 2, 2, 2, 3, 3, 3, 3, 0, 1]:
        p.begin_layer()
        seq.append(p.lookup(0, e))
    paths = [s[0] for s in seq]
    # 0, 1 take the free slots; 2 rides scratch for its first touch and two
    # RAM hits, then is promoted, evicting the LRU (0); 3 likewise evicts 1;
    # 0 and 1 come back as first RAM hits -> scratch
    assert paths == [3, 3, 4, 1, 1, 2, 4, 1, 1, 2, 1, 1], paths
    assert seq[5][2] == (0, 0)      # promoting 2 evicted expert 0
    assert seq[9][2] == (0, 1)      # promoting 3 evicted expert 1
    assert seq[5][1] == seq[0][1]   # and took its slot
    st = p.stats()
    assert (st["lookups"], st["vram_hits"], st["promotions"], st["evictions"]) == (12, 0, 2, 2)
    # the scratch ring is round robin over its 3 slots
    scratch_slots = [s[1] for s in seq if s[0] in (1, 4)]
    assert scratch_slots == [0, 1, 2, 0, 1, 2, 0, 1]


def test_vram_hit_refreshes_recency():
    p = tier.Policy(1, 5, 2, 2, promote_hits=1)
    for e in (0, 1):
        p.begin_layer()
        assert p.lookup(0, e)[0] == tier.COLD_VRAM
    p.begin_layer()
    assert p.lookup(0, 0)[0] == tier.VRAM_HIT      # 0 is now MRU, 1 is LRU
    p.begin_layer()
    assert p.lookup(0, 2)[0] == tier.COLD_SCRATCH
    p.begin_layer()
    path, _, victim = p.lookup(0, 2)                # promote_hits = 1
    assert path == tier.RAM_PROMOTE and victim == (0, 1)


def test_experts_of_the_current_layer_are_never_evicted():
    # 2 slots, both filled by this layer's first two experts: the third
    # expert's promotion finds no evictable slot and rides scratch instead
    p = tier.Policy(1, 3, 2, 4, promote_hits=1)
    p.begin_layer()
    for e in (0, 1, 2):
        p.lookup(0, e)
    p.begin_layer()
    assert p.lookup(0, 0)[0] == tier.VRAM_HIT
    assert p.lookup(0, 1)[0] == tier.VRAM_HIT
    assert p.lookup(0, 2)[0] == tier.RAM_SCRATCH    # 0 and 1 are pinned by this layer
    p.begin_layer()
    path, _, victim = p.lookup(0, 2)                # next layer: LRU (0) is evictable
    assert path == tier.RAM_PROMOTE and victim == (0, 0)


def test_bad_arguments():
    with pytest.raises(ValueError):
        tier.Policy(0, 4, 2, 2)
    p = tier.Policy(2, 4, 2, 2)
    with pytest.raises(ValueError):
        p.lookup(2, 0)
    with pytest.raises(ValueError):
        p.lookup(0, 4)
