"""The reference's CPU dequant + matmul path, in torch CPU ops (cpu_baseline leg).

TEST/BENCH INFRASTRUCTURE ONLY (see oracle/wlq_oracle.py): imported by
bench.py's cpu_baseline leg and tests, never by the product.

Follows the reference's host-side reconstruction and forward semantics:
unpack the row-aligned codes, dequantize with torch.gather over the fp16 LUT
(vllm_wlq/linear_method.py:609-610, :880-881), overwrite outliers with the fp16
bits ``u8 << 8`` (:611-623, :882-888), then ``y = x.float() @ W0.float().T`` and
the DoRA epilogue ``(y + s * fp16(x A^T).float() @ B^T) * gamma`` rounded to
fp16 (:937-1009 with the GEMV epilogue csrc/gemv_kernel.cu:309-317).  Group
LUTs index lut[n, k // G, code].
"""
from __future__ import annotations

import time
from typing import Optional

import numpy as np
import torch


class CpuLayer:
    """Device-format layer held as CPU tensors."""

    def __init__(self, L):
        self.N, self.K, self.bits, self.G = L.N, L.K, L.bits, L.group_size
        self.wpr = L.wpr
        self.q = torch.from_numpy(L.q.view(np.int32).copy())
        self.lut = torch.from_numpy(L.lut.reshape(L.N, -1).copy())
        self.offsets = L.offsets
        self.cols = L.cols
        self.vals = torch.from_numpy(L.vals.copy())
        self.A = None if L.A is None else torch.from_numpy(L.A.copy())
        self.B = None if L.B is None else torch.from_numpy(L.B.copy())
        self.gamma = None if L.gamma is None else torch.from_numpy(L.gamma.copy())
        self.s = L.lora_scale
        # outlier coordinates (row, global column), expanded once like the reference's loader
        nch = self.offsets.shape[1] - 1
        chunk = 640 if self.bits == 3 else 512
        counts = np.diff(self.offsets, axis=1).astype(np.int64)
        rows = np.repeat(np.repeat(np.arange(self.N), nch), counts.ravel())
        chunk_idx = np.repeat(np.tile(np.arange(nch), self.N), counts.ravel())
        gcols = chunk_idx * chunk + self.cols.astype(np.int64)
        keep = gcols < self.K
        self.o_rows = torch.from_numpy(rows[keep])
        self.o_cols = torch.from_numpy(gcols[keep])
        self.o_vals = (self.vals[torch.from_numpy(np.flatnonzero(keep))].to(torch.int32) << 8).to(torch.int16).view(
            torch.float16)


def dequant(layer: CpuLayer) -> torch.Tensor:
    spw = 10 if layer.bits == 3 else 32 // layer.bits
    mask = (1 << layer.bits) - 1
    words = layer.q.view(layer.N, layer.wpr).to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(spw, dtype=torch.int64) * layer.bits
    codes = ((words[:, :, None] >> shifts) & mask).reshape(layer.N, -1)[:, :layer.K]
    if layer.G > 0 and layer.G < layer.K:
        codes = codes + (torch.arange(layer.K) // layer.G)[None, :] * (1 << layer.bits)
    W0 = torch.gather(layer.lut, 1, codes)
    if layer.o_rows.numel():
        W0[layer.o_rows, layer.o_cols] = layer.o_vals
    return W0


def forward(layer: CpuLayer, x: torch.Tensor, W0: Optional[torch.Tensor] = None) -> torch.Tensor:
    if W0 is None:
        W0 = dequant(layer)
    y = x.float() @ W0.float().T
    if layer.B is not None:
        H = (x.float() @ layer.A.float().T).half().float()
        y = (y + layer.s * (H @ layer.B.float().T)) * layer.gamma.float()
    return y.half()


def time_layers(layers, x_by_k, reps: int = 2):
    """Median seconds per pass over ``layers`` for (dequant+matmul per call, matmul with cached W0)."""
    full, cached = [], []
    W0s = [dequant(l) for l in layers]
    for _ in range(reps):
        t = time.perf_counter()
        for l in layers:
            forward(l, x_by_k[l.K])
        full.append(time.perf_counter() - t)
        t = time.perf_counter()
        for l, W in zip(layers, W0s):
            forward(l, x_by_k[l.K], W)
        cached.append(time.perf_counter() - t)
    return float(np.median(full)), float(np.median(cached))
