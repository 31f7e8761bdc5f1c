"""Seeded synthetic workloads for the int4 MoE expert path.

Shapes follow the reference's model constants (wisp/models/constants.py):
Mixtral-8x7B hidden 4096 / inter 14336 / 8 experts / top-2 (softmax router),
DeepSeek-V3 hidden 7168 / routed inter 2048 / 256 experts / top-8 plus one
shared expert of inter 2048 (sigmoid router). Weights are int4 with group
size 128 and fp16 scales ~ |N(0, 0.01)|; nibbles are uniform in 0..15
(so q - 8 is uniform in [-8, 7]); zeros are +0 unless requested.

Blobs use the reference expert-file layout (wisp/converter/partitioner.py:
11-27, csrc/core/wisp_engine.h:214-238): a 120-byte header, then for gate,
up, down in order [packed][scales][zeros].
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

MAGIC = 0x57455850
HEADER = struct.Struct("<6I")
MAT_HEADER = struct.Struct("<2I3Q")
HEADER_BYTES = HEADER.size + 3 * MAT_HEADER.size  # 120


@dataclass(frozen=True)
class MoeShape:
    name: str
    hidden: int
    inter: int
    n_experts: int
    top_k: int
    group_size: int = 128
    router: str = "softmax"   # or "sigmoid"
    shared: bool = False


MIXTRAL = MoeShape("mixtral-8x7b", 4096, 14336, 8, 2, 128, "softmax", False)
DSV3 = MoeShape("deepseek-v3", 7168, 2048, 256, 8, 128, "sigmoid", True)


def mat_shapes(inter: int, hidden: int):
    """(rows, cols) of gate, up, down."""
    return [(inter, hidden), (inter, hidden), (hidden, inter)]


def blob_size(inter: int, hidden: int, gs: int) -> int:
    total = HEADER_BYTES
    for r, c in mat_shapes(inter, hidden):
        n = r * c
        total += (n + 1) // 2 + 2 * (2 * ((n + gs - 1) // gs))
    return total


def expert_bytes_no_zeros(inter: int, hidden: int, gs: int) -> int:
    """Algorithmic bytes of one expert: packed + scales (zeros excluded)."""
    return sum((r * c) // 2 + 2 * (r * c // gs) for r, c in mat_shapes(inter, hidden))


def write_header(buf: np.ndarray, layer: int, expert: int, inter: int, hidden: int, gs: int):
    hdr = HEADER.pack(MAGIC, 1, layer, expert, gs, 3)
    for r, c in mat_shapes(inter, hidden):
        n = r * c
        ng = (n + gs - 1) // gs
        hdr += MAT_HEADER.pack(r, c, (n + 1) // 2, 2 * ng, 2 * ng)
    buf[:HEADER_BYTES] = np.frombuffer(hdr, dtype=np.uint8)


def section_offsets(inter: int, hidden: int, gs: int):
    """[(packed_off, scales_off, zeros_off, rows, cols)] per matrix."""
    out, off = [], HEADER_BYTES
    for r, c in mat_shapes(inter, hidden):
        n = r * c
        ng = (n + gs - 1) // gs
        p = off
        s = p + (n + 1) // 2
        z = s + 2 * ng
        off = z + 2 * ng
        out.append((p, s, z, r, c))
    return out


def make_blob(rng: np.random.Generator, inter: int, hidden: int, gs: int = 128,
              layer: int = 0, expert: int = 0, zeros: bool = False,
              out: np.ndarray | None = None) -> np.ndarray:
    """One expert blob (uint8). Nibbles uniform 0..15; scales fp16(|N(0,.01)|);
    zeros +0, or fp16(N(0, .01)) when `zeros`."""
    size = blob_size(inter, hidden, gs)
    buf = np.empty(size, dtype=np.uint8) if out is None else out[:size]
    write_header(buf, layer, expert, inter, hidden, gs)
    for (p, s, z, r, c) in section_offsets(inter, hidden, gs):
        n = r * c
        ng = (n + gs - 1) // gs
        buf[p:s] = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
        sc = np.abs(rng.standard_normal(ng, dtype=np.float32) * 0.01).astype(np.float16)
        buf[s:z] = sc.view(np.uint8)
        if zeros:
            zz = (rng.standard_normal(ng, dtype=np.float32) * 0.01).astype(np.float16)
        else:
            zz = np.zeros(ng, dtype=np.float16)
        buf[z:z + 2 * ng] = zz.view(np.uint8)
    return buf


def blob_views(blob: np.ndarray, inter: int, hidden: int, gs: int):
    """[(packed u8, scales u16, zeros u16, rows, cols)] views into a blob."""
    res = []
    for (p, s, z, r, c) in section_offsets(inter, hidden, gs):
        n = r * c
        ng = (n + gs - 1) // gs
        res.append((blob[p:s], blob[s:z].view(np.uint16), blob[z:z + 2 * ng].view(np.uint16), r, c))
    return res


def make_x(rng: np.random.Generator, n_tokens: int, hidden: int) -> np.ndarray:
    """fp16 N(0, 1) activations [n_tokens, hidden]."""
    return rng.standard_normal((n_tokens, hidden), dtype=np.float32).astype(np.float16)


def make_router(rng: np.random.Generator, n_experts: int, hidden: int, std: float = 0.02) -> np.ndarray:
    return (rng.standard_normal((n_experts, hidden), dtype=np.float32) * std).astype(np.float16)


def uniform_topk(rng: np.random.Generator, n_tokens: int, n_experts: int, top_k: int) -> np.ndarray:
    """top_k distinct experts per token, uniformly at random [n_tokens, top_k]."""
    return np.stack([rng.choice(n_experts, size=top_k, replace=False)
                     for _ in range(n_tokens)]).astype(np.int32)


def zipf_topk(rng: np.random.Generator, n_tokens: int, n_experts: int, top_k: int,
              s: float = 1.1) -> np.ndarray:
    """top_k distinct experts per token drawn without replacement from
    P(e) proportional to (e + 1)^-s [n_tokens, top_k]."""
    p = 1.0 / np.arange(1, n_experts + 1, dtype=np.float64) ** s
    p /= p.sum()
    return np.stack([rng.choice(n_experts, size=top_k, replace=False, p=p)
                     for _ in range(n_tokens)]).astype(np.int32)


def route_weights(rng: np.random.Generator, n_tokens: int, top_k: int) -> np.ndarray:
    """Positive weights that sum to 1 per token [n_tokens, top_k] (fp32)."""
    w = rng.random((n_tokens, top_k), dtype=np.float32) + 0.5
    return (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


def slot_stride(inter: int, hidden: int, gs: int) -> int:
    """Bytes per expert slot in a device arena: the blob sits at slot + 8 so
    that every section (120 + 16k bytes into the blob) is 16-byte aligned."""
    b = blob_size(inter, hidden, gs) + 8
    return (b + 4095) // 4096 * 4096


# Seeds of the benchmark workloads (the config-scale tests reuse them).
PREFILL_SEED = 2048
DSV3_BENCH_SEED = 777
MIXTRAL_BENCH_SEED = 1234


def bench_expert(shape: MoeShape, seed: int, set_idx: int, e: int,
                 out: np.ndarray | None = None) -> np.ndarray:
    """Routed expert e of benchmark expert set set_idx."""
    return make_blob(np.random.default_rng([seed, set_idx, e]), shape.inter, shape.hidden,
                     shape.group_size, expert=e, out=out)


def bench_shared(shape: MoeShape, seed: int, set_idx: int,
                 out: np.ndarray | None = None) -> np.ndarray:
    """The shared expert of benchmark set set_idx."""
    return make_blob(np.random.default_rng([seed, 99999, set_idx]), shape.inter, shape.hidden,
                     shape.group_size, expert=99999, out=out)


def prefill_draw(shape: MoeShape, n_tokens: int, seed: int = PREFILL_SEED):
    """The prefill workload's inputs: top-k routing drawn without replacement
    from Zipf(1.1) over the routed experts, positive weights summing to 1,
    and fp16 N(0, 1) tokens, in that order from one generator."""
    rng = np.random.default_rng(seed)
    idx = zipf_topk(rng, n_tokens, shape.n_experts, shape.top_k)
    w = route_weights(rng, n_tokens, shape.top_k)
    x = make_x(rng, n_tokens, shape.hidden)
    return idx, w, x


def streaming_draw(shape: MoeShape, n_layers: int, steps: int, seed: int = 55, n_x: int = 16):
    """The expert-streaming workload's inputs: a pool of n_x fp16 tokens, then
    per step and layer one token's Zipf(1.1) top-k routing and weights.
    Returns (x [n_x, hidden], routes[step][layer] [1, top_k],
    weights[step][layer] [1, top_k])."""
    rng = np.random.default_rng(seed)
    xs = make_x(rng, n_x, shape.hidden)
    routes = [[zipf_topk(rng, 1, shape.n_experts, shape.top_k) for _ in range(n_layers)]
              for _ in range(steps)]
    weights = [[route_weights(rng, 1, shape.top_k) for _ in range(n_layers)]
               for _ in range(steps)]
    return xs, routes, weights
