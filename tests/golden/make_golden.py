"""Writes tests/golden/wlq_small.npz: a small seeded WLQ layer in the reference's
formats (row-aligned 4-bit and 3-bit codes, group and per-row fp16 LUTs, chunk CSR
with e5m2 values, DoRA factors) with the oracle's outputs: W0 bits and y at M=1 and
M=16 (reference rounding points).

The reference ships no golden vectors and cannot run here, so these are vectors of
this build's oracle (itself pinned by hand-computed and brute-force checks); they
freeze its results for regression and give the GPU tests fixed inputs.

Run: python tests/golden/make_golden.py  (from the repository root)
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import wlq_oracle as O  # noqa: E402
from qwen_wlqfastshot_helen_beta_amd import synth  # noqa: E402


def main():
    out = {}
    for tag, bits, gs in (("b4g128", 4, 128), ("b3row", 3, 0)):
        L = synth.make_layer(N=32, K=680, bits=bits, group_size=gs, rank=8, density=0.01, seed=2024, heavy_frac=0.2,
                             heavy_mult=10.0)
        W0 = O.dequant(L.q, L.lut, L.N, L.K, bits, L.offsets, L.cols, L.vals, group_size=gs)
        x1 = synth.make_activations(1, L.K, seed=1)
        x16 = synth.make_activations(16, L.K, seed=16)
        y1 = O.apply(x1, W0, L.A, L.B, L.gamma, L.lora_scale)
        y16 = O.apply(x16, W0, L.A, L.B, L.gamma, L.lora_scale)
        for k, v in dict(q=L.q, lut=L.lut, offsets=L.offsets, cols=L.cols, vals=L.vals, A=L.A, B=L.B,
                         gamma=L.gamma, x1=x1, x16=x16, W0=W0, y1=y1, y16=y16,
                         meta=np.array([L.N, L.K, bits, gs, L.wpr], np.int64)).items():
            out[f"{tag}_{k}"] = v
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "wlq_small.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
