"""Writes the golden fixtures in tests/golden/ (run once, in a tree where the
reference's scalar CPU path was compiled into oracle/_ref).

Every expected output here is produced by the REFERENCE's own C code
(csrc/core/wisp_engine.c, compiled from its sources by oracle/Makefile):
  dequant_g64.npz     wisp_debug_expert_probe        (wisp_engine.c:311-349)
  gemv_int4.npz       cpu_gemv_int4, scalar branch   (wisp_engine.c:822-845)
  expert_ffn.npz      cpu_expert_ffn                 (wisp_engine.c:1534-1561)
  router_softmax.npz  cpu_router_topk                (wisp_engine.c:782-818)
  layer_ops.npz       cpu_rmsnorm, cpu_gemv_t_f16,   (wisp_engine.c:647-675)
                      cpu_residual_add
The fp16 column of dequant_g64 is the fp32 probe value rounded to nearest
even, which is what the reference GPU kernel stores
(csrc/cuda/expert_loader.cu:42).

Usage: python tests/golden/make_golden.py
"""
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402
from wisp_amd import synth  # noqa: E402


def main():
    R = O.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libwisp_ref.so is not built (needs the reference tree)")
    rng = np.random.default_rng(20260101)

    # dequant, g64, nonzero zeros: 2 x 128 elements of gate via the C probe
    inter, hidden, gs = 16, 128, 64
    blob = synth.make_blob(rng, inter, hidden, gs, zeros=True)
    p, s, z, r, c = synth.blob_views(blob, inter, hidden, gs)[0]
    n = r * c
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "L000_E00000.bin")
        with open(path, "wb") as f:
            f.write(blob.tobytes())
        out = np.empty(n, np.float32)
        assert R.ref_debug_probe(path.encode(), 0, n, O._p(out)) == 0
    np.savez_compressed(os.path.join(HERE, "dequant_g64.npz"), packed=p.copy(), scales=s.copy(),
                        zeros=z.copy(), n=n, gs=gs, out_f32=out,
                        out_f16=out.astype(np.float16).view(np.uint16))

    # gemv_int4 on a [96, 512] g128 matrix with nonzero zeros
    rows, cols, gs = 96, 512, 128
    packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    scales = (np.abs(rng.standard_normal(rows * cols // gs)) * 0.01).astype(np.float16).view(np.uint16)
    zeros = (rng.standard_normal(rows * cols // gs) * 0.01).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(cols).astype(np.float16).astype(np.float32)
    y = np.empty(rows, np.float32)
    R.ref_gemv_int4(O._p(packed), O._p(scales), O._p(zeros), O._p(x), O._p(y), rows, cols, gs)
    np.savez_compressed(os.path.join(HERE, "gemv_int4.npz"), packed=packed, scales=scales,
                        zeros=zeros, x=x, y=y, rows=rows, cols=cols, gs=gs)

    # one expert FFN (inter 256, hidden 512, g128, zeros) accumulated with w
    inter, hidden, gs = 256, 512, 128
    blob = synth.make_blob(rng, inter, hidden, gs, zeros=True)
    x = rng.standard_normal(hidden).astype(np.float16).astype(np.float32)
    acc = rng.standard_normal(hidden).astype(np.float32)
    out = acc.copy()
    assert R.ref_expert_ffn(O._p(blob), blob.nbytes, O._p(x), O._p(out), np.float32(0.625)) == 0
    np.savez_compressed(os.path.join(HERE, "expert_ffn.npz"), blob=blob, x=x, acc=acc, w=0.625,
                        out=out, inter=inter, hidden=hidden, gs=gs)

    # softmax router, 64 experts, hidden 512, top-8, with bias
    n_exp, hidden, k = 64, 512, 8
    W = synth.make_router(rng, n_exp, hidden)
    bias = (rng.standard_normal(n_exp) * 0.1).astype(np.float16)
    x = rng.standard_normal(hidden).astype(np.float16).astype(np.float32)
    idx = np.empty(k, np.int32); w = np.empty(k, np.float32); lg = np.empty(n_exp, np.float32)
    R.ref_router_topk(O._p(W), O._p(bias), O._p(x), O._p(lg), n_exp, hidden, k, O._p(idx), O._p(w))
    np.savez_compressed(os.path.join(HERE, "router_softmax.npz"), W=W.view(np.uint16),
                        bias=bias.view(np.uint16), x=x, k=k, idx=idx, w=w, probs=lg)
    # the decode step's neighbouring ops: RMSNorm (eps 1e-6, n 7168),
    # transposed fp16 GEMV [96, 512], residual add
    rng2 = np.random.default_rng(20261203)
    n = 7168
    x = (rng2.standard_normal(n) * 3.0).astype(np.float32)
    wn = (1.0 + 0.1 * rng2.standard_normal(n)).astype(np.float16)
    y = np.empty(n, np.float32)
    R.ref_rmsnorm(O._p(x), O._p(wn), O._p(y), n, np.float32(1e-6))
    rows, cols = 96, 512
    Wt = (rng2.standard_normal((rows, cols)) * 0.05).astype(np.float16)
    xt = rng2.standard_normal(rows).astype(np.float32)
    yt = np.empty(cols, np.float32)
    R.ref_gemv_t_f16(O._p(Wt), O._p(xt), O._p(yt), rows, cols)
    r0 = rng2.standard_normal(n).astype(np.float32)
    d = rng2.standard_normal(n).astype(np.float32)
    r1 = r0.copy()
    R.ref_residual_add(O._p(r1), O._p(d), n)
    np.savez_compressed(os.path.join(HERE, "layer_ops.npz"), x=x, w=wn.view(np.uint16), eps=1e-6,
                        y=y, Wt=Wt.view(np.uint16), xt=xt, yt=yt, r0=r0, d=d, r1=r1)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
