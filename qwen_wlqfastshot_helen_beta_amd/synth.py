"""Seeded synthetic WLQ layers (the workloads of the benchmark configs).

One generator feeds tests and benchmarks, so GPU and CPU see identical inputs.

* codes: uniform integers in [0, 2**bits);
* LUTs: for each (row, group) 128 draws of N(0, sigma) are fitted by least
  squares with a ``terms``-term metalog quantile function (Keelin 2016, "The
  Metalog Distributions", Decision Analysis 13(4), eq. 6 basis
  1, L, (y-.5)L, (y-.5), (y-.5)^2, (y-.5)^2 L, ... with L = ln(y/(1-y)),
  fitted at the plotting positions y_i = (i - 0.5)/n of the sorted draws),
  evaluated at y_j = (j + 0.5)/2**bits, sorted, rounded to fp16;
* outliers: exactly round(d*N*K) positions without replacement, optionally with
  a fraction of "heavy" rows drawing ``heavy_mult`` times the per-row rate of the
  others at the same total density; values N(0, 0.2) -> fp16 -> e5m2 bytes;
* DoRA: A [r, K], B [N, r] ~ N(0, 0.01) in fp16, lora_alpha = r (scale 1), and
  gamma = m / ||W0 + s B A||_row with m = U(0.9, 1.1) * ||W0 + s B A||_row, i.e.
  gamma = fp16(U(0.9, 1.1));
* activations: fp16 N(0, 1).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np

from . import formats

# Qwen2.5-7B linear shapes (out x in) and Qwen2.5-0.5B up_proj.
QWEN25_7B_SHAPES: Dict[str, tuple] = {
    "q_proj": (3584, 3584),
    "k_proj": (512, 3584),
    "v_proj": (512, 3584),
    "o_proj": (3584, 3584),
    "gate_proj": (18944, 3584),
    "up_proj": (18944, 3584),
    "down_proj": (3584, 18944),
}
QWEN25_05B_UP_PROJ = (4864, 896)


def metalog_basis(y: np.ndarray, terms: int) -> np.ndarray:
    """Keelin metalog basis functions evaluated at probabilities ``y`` -> [len(y), terms]."""
    y = np.asarray(y, dtype=np.float64)
    L = np.log(y / (1.0 - y))
    c = y - 0.5
    cols = []
    for j in range(1, terms + 1):
        if j == 1:
            cols.append(np.ones_like(y))
        elif j == 2:
            cols.append(L)
        elif j == 3:
            cols.append(c * L)
        elif j == 4:
            cols.append(c)
        elif j % 2 == 1:  # 5, 7, ...: (y-.5)^((j-1)/2)
            cols.append(c ** ((j - 1) // 2))
        else:  # 6, 8, ...: (y-.5)^(j/2-1) * L
            cols.append(c ** (j // 2 - 1) * L)
    return np.stack(cols, axis=1)


def metalog_lut_projector(bits: int, samples: int = 128, terms: int = 4) -> np.ndarray:
    """Matrix P [2**bits, samples]: LUT = P @ sorted(samples) (fit then evaluate)."""
    yi = (np.arange(1, samples + 1) - 0.5) / samples
    Y = metalog_basis(yi, terms)
    yq = (np.arange(1 << bits) + 0.5) / (1 << bits)
    return metalog_basis(yq, terms) @ np.linalg.pinv(Y)


def metalog_luts(rng: np.random.Generator, n_luts: int, bits: int, sigma: float = 0.02,
                 samples: int = 128, terms: int = 4) -> np.ndarray:
    """``n_luts`` sorted fp16 LUTs of 2**bits entries -> float16 [n_luts, 2**bits]."""
    P = metalog_lut_projector(bits, samples, terms).astype(np.float32)
    out = np.empty((n_luts, 1 << bits), dtype=np.float16)
    step = 1 << 16
    for s in range(0, n_luts, step):
        n = min(step, n_luts - s)
        draws = rng.standard_normal((n, samples), dtype=np.float32) * np.float32(sigma)
        draws.sort(axis=1)
        out[s:s + n] = np.sort(draws @ P.T, axis=1).astype(np.float16)
    return out


@dataclass
class SynthLayer:
    N: int
    K: int
    bits: int
    group_size: int
    wpr: int
    q: np.ndarray            # int32 [N * wpr]
    lut: np.ndarray          # float16 [N, 2**bits] (group_size 0) or [N, ng, 2**bits]
    offsets: np.ndarray      # int32 [N, nch+1]
    cols: np.ndarray         # uint16 [nnz]
    vals: np.ndarray         # uint8 [nnz]
    A: Optional[np.ndarray]  # float16 [r, K]
    B: Optional[np.ndarray]  # float16 [N, r]
    gamma: Optional[np.ndarray]  # float16 [N]
    lora_scale: float = 1.0
    meta: dict = field(default_factory=dict)

    @property
    def rank(self) -> int:
        return 0 if self.B is None else int(self.B.shape[1])

    @property
    def nnz(self) -> int:
        return int(self.cols.size)

    def codes(self) -> np.ndarray:
        """Unpacked codes [N, K] (uint8), for checkers."""
        spw = formats.symbols_per_word(self.bits)
        k = np.arange(self.K)
        words = self.q.view(np.uint32).reshape(self.N, self.wpr)[:, k // spw]
        return ((words >> ((k % spw) * self.bits).astype(np.uint32)) & np.uint32((1 << self.bits) - 1)).astype(np.uint8)

    def headline_bytes(self) -> int:
        """Code + LUT + outlier bytes streamed per call (the GEMV headline traffic)."""
        nch = formats.num_chunks(self.K, self.bits)
        return int(self.q.nbytes + self.lut.nbytes + self.nnz * 3 + self.N * (nch + 1) * 4)

    def aux_bytes(self, M: int) -> int:
        """x, y and DoRA bytes (reported separately from the headline)."""
        r = self.rank
        return int(M * self.K * 2 + M * self.N * 2 + r * self.K * 2 + self.N * r * 2 + (self.N * 2 if r else 0))

    def to_torch(self, device="cuda"):
        import torch
        d = {
            "q_packed": torch.from_numpy(self.q.view(np.int32)).to(device),
            "lut_c": torch.from_numpy(self.lut).to(device),
            "chunk_offsets": torch.from_numpy(self.offsets).to(device),
            "chunk_cols": torch.from_numpy(self.cols.view(np.int16)).to(device).view(torch.uint16),
            "chunk_vals": torch.from_numpy(self.vals).to(device),
        }
        if self.B is not None:
            d["lora_A"] = torch.from_numpy(self.A).to(device)
            d["lora_B"] = torch.from_numpy(self.B).to(device)
            d["dora_gamma"] = torch.from_numpy(self.gamma).to(device)
        return d


def _outlier_positions(rng, N, K, nnz, heavy_frac, heavy_mult):
    if nnz == 0:
        z = np.zeros(0, dtype=np.int64)
        return z, z
    if heavy_frac <= 0:
        flat = np.sort(rng.choice(N * K, size=nnz, replace=False))
        return flat // K, flat % K
    n_heavy = int(round(heavy_frac * N))
    heavy = np.zeros(N, dtype=bool)
    heavy[rng.choice(N, size=n_heavy, replace=False)] = True
    weight = np.where(heavy, float(heavy_mult), 1.0)
    ideal = nnz * weight / weight.sum()
    counts = np.minimum(np.floor(ideal).astype(np.int64), K)
    rem = nnz - int(counts.sum())
    if rem > 0:  # hand the remainder to rows by largest fractional part, then randomly
        frac = ideal - np.floor(ideal)
        order = np.lexsort((rng.random(N), -frac))
        for r in order:
            if rem == 0:
                break
            if counts[r] < K:
                counts[r] += 1
                rem -= 1
    rows, cols = [], []
    for r in range(N):
        c = int(counts[r])
        if c:
            cs = np.sort(rng.choice(K, size=c, replace=False))
            rows.append(np.full(c, r, dtype=np.int64))
            cols.append(cs.astype(np.int64))
    return np.concatenate(rows), np.concatenate(cols)


def make_layer(N: int, K: int, bits: int = 4, group_size: int = 128, rank: int = 16,
               density: float = 0.005, seed: int = 0, heavy_frac: float = 0.0, heavy_mult: float = 10.0,
               lut_sigma: float = 0.02) -> SynthLayer:
    """Build one synthetic WLQ layer (see module docstring)."""
    rng = np.random.default_rng(seed)
    ng = formats.num_groups(K, group_size)
    codes = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint8)
    q, wpr = formats.pack_indices_row_aligned(codes, bits)
    del codes
    lut = metalog_luts(rng, N * ng, bits, sigma=lut_sigma)
    lut = lut.reshape(N, 1 << bits) if group_size <= 0 else lut.reshape(N, ng, 1 << bits)
    nnz = int(round(density * N * K))
    rows, cols = _outlier_positions(rng, N, K, nnz, heavy_frac, heavy_mult)
    chunk = formats.chunk_width(bits)
    offsets, ccols, order = formats.chunk_csr_from_coords(rows, cols, N, K, chunk)
    vals = formats.fp16_to_e5m2_u8(rng.normal(0.0, 0.2, size=rows.size).astype(np.float16))[order]
    A = B = gamma = None
    if rank > 0:
        A = (rng.standard_normal((rank, K), dtype=np.float32) * 0.01).astype(np.float16)
        B = (rng.standard_normal((N, rank), dtype=np.float32) * 0.01).astype(np.float16)
        gamma = rng.uniform(0.9, 1.1, size=N).astype(np.float16)
    return SynthLayer(N=N, K=K, bits=bits, group_size=group_size, wpr=wpr, q=q.view(np.int32), lut=lut,
                      offsets=offsets, cols=ccols, vals=vals, A=A, B=B, gamma=gamma, lora_scale=1.0,
                      meta=dict(seed=seed, density=density, heavy_frac=heavy_frac, heavy_mult=heavy_mult))


def merge_layers(parts) -> SynthLayer:
    """Output-dimension merge of layers sharing K (vLLM's qkv_proj / gate_up_proj):
    rows concatenated, CSR offsets rebased, DoRA A stacked along the rank and B
    block-diagonal, as the plugin's loader merges shards."""
    p0 = parts[0]
    assert all(p.K == p0.K and p.bits == p0.bits and p.group_size == p0.group_size for p in parts)
    offs, base = [], 0
    for p in parts:
        offs.append(p.offsets.astype(np.int64) + base)
        base += p.nnz
    N = sum(p.N for p in parts)
    A = B = gamma = None
    if all(p.B is not None for p in parts):
        A = np.concatenate([p.A for p in parts], axis=0)
        R = sum(p.rank for p in parts)
        B = np.zeros((N, R), dtype=np.float16)
        r0 = c0 = 0
        for p in parts:
            B[r0:r0 + p.N, c0:c0 + p.rank] = p.B
            r0 += p.N
            c0 += p.rank
        gamma = np.concatenate([p.gamma for p in parts])
    return SynthLayer(N=N, K=p0.K, bits=p0.bits, group_size=p0.group_size, wpr=p0.wpr,
                      q=np.concatenate([p.q for p in parts]), lut=np.concatenate([p.lut for p in parts]),
                      offsets=np.concatenate(offs).astype(np.int32), cols=np.concatenate([p.cols for p in parts]),
                      vals=np.concatenate([p.vals for p in parts]), A=A, B=B, gamma=gamma,
                      lora_scale=p0.lora_scale, meta=dict(merged=len(parts)))


def make_activations(M: int, K: int, seed: int = 1) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
