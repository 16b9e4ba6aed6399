"""Writes the golden fixtures in this directory from the reference's own C.

Run in a container that holds the reference sources (/root/reference):
    make -C oracle && python tests/golden/gen_golden.py
The reference is compiled by oracle/Makefile into oracle/_ref/libqkref.so
from its unmodified sources (slm/tensor.c, simd/*.c via slm/qwen.c). The
fixtures are data only: inputs, and the outputs the reference computed for
them. Separate-epilogue outputs come from the reference's scalar tier
(simd/quants.h), fused-epilogue outputs from its AVX2-FMA tier
(simd/avx.c); both are evaluated on this container's CPU.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
from conftest import oracle, synth  # noqa: E402
from cases import edge_rows  # noqa: E402

REF_FILES = ["simd/quants.h", "simd/avx.c", "simd/simd.c", "slm/tensor.c", "slm/model.c", "slm/sampler.c"]


def main(refroot="/root/reference"):
    R = oracle.Ref()
    assert 2 in R.tiers(), "fixtures need the AVX2-FMA tier on this CPU"
    shas = {f: hashlib.sha256(open(os.path.join(refroot, f), "rb").read()).hexdigest() for f in REF_FILES}
    meta = dict(seed=0, ref_label=R.label(), **{"sha256:" + k: v for k, v in shas.items()})
    k = 512
    x = np.concatenate([edge_rows(k), synth.activations(5, k, seed=0, tag=3)])
    np.savez_compressed(os.path.join(HERE, "quant.npz"), x=x, q8k=R.quantize_q8k(x),
                        q8_0=R.quantize_q8_0(x), meta=np.array(repr(meta)))
    out = {"meta": np.array(repr(meta))}
    for wt, name in ((12, "q4k"), (13, "q5k"), (14, "q6k"), (8, "q8_0")):
        w = synth.blocks(wt, 8, k, seed=0, tag=wt)
        # random rows, then all-zero and ~1e37 rows (8-lane sum overflow)
        xs = np.concatenate([synth.activations(3, k, seed=0, tag=wt + 1), edge_rows(k)[[0, 6]]])
        xq = R.quantize_for(wt, xs)
        for tier, tag in ((0, "sep"), (2, "fused")):
            y = np.array([[R.row_dot(wt, w[j], xq[t], k, tier) for j in range(8)] for t in range(xs.shape[0])],
                         np.float32)
            out[f"{name}_y_{tag}"] = y
        out[f"{name}_w"] = w
        out[f"{name}_x"] = xs
        out[f"{name}_xq"] = xq
        if wt != 8:
            out[f"{name}_deq"] = R.dequant(wt, w, w.size // {12: 144, 13: 176, 14: 210}[wt])
    np.savez_compressed(os.path.join(HERE, "dots.npz"), **out)
    rng = np.random.default_rng(7)
    v = rng.normal(0, 1, 5000).astype(np.float32)
    v[[10, 4000]] = 9.5                       # tied maximum: first index wins
    v[[20, 30, 40]] = 5.25                    # ties below the top
    am = R.argmax(v)
    ti, tv = R.topk_collect(v, 40)
    np.savez_compressed(os.path.join(HERE, "select.npz"), v=v, argmax=np.int32(am), topk_idx=ti, topk_val=tv,
                        meta=np.array(repr(meta)))
    print("wrote fixtures;", meta["ref_label"])


if __name__ == "__main__":
    main()
