"""GPU parity at the full Qwen2.5-7B shapes on the paths the benchmark times.

* Config 1 (decode, M = 1, 4, 8, 16, 32): the prepared-layout product (what
  ``WLQLinearMethod.apply`` runs once a layer is loaded) at vLLM's merged
  projections -- qkv_proj 4608x3584 (DoRA rank 48: q|k|v adapters stacked),
  o_proj 3584x3584, gate_up_proj 37888x3584 (rank 32), down_proj 3584x18944 --
  and at the seven unmerged shapes, 4-bit, LUT group 128, 0.5% outliers, DoRA H
  computed inside the kernel from lora_A.
* Config 2 (prefill, M = 128, 512, 2048, 8192): the seven shapes through the
  same op with the prepared buffer passed, as apply() does (M > 32 runs the
  MFMA GEMM).

Outputs are checked on a subset of output rows (random rows, the densest outlier
rows and both edge rows) against the fp64 oracle built from those rows' codes,
LUTs and CSR entries, so the CPU side stays at seconds per case.  Both rounding
conventions are checked where they differ (M >= 16).  Tolerance: TOLERANCE in
gpu_helpers (max |rel err| <= 2e-3 and 2 fp16 ulp elementwise)."""
from __future__ import annotations

import functools

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, check_rows, pick_rows, run_prepared
from oracle import wlq_oracle as O
from qwen_wlqfastshot_helen_beta_amd import synth

pytestmark = pytest.mark.gpu

SHAPES = synth.QWEN25_7B_SHAPES
NAMES = list(SHAPES)


def _case(msg):
    print(f"[case] {msg}", flush=True)


@functools.lru_cache(maxsize=None)
def unmerged(name: str) -> synth.SynthLayer:
    """The benchmark's layers: 4-bit, G = 128, r = 16, d = 0.5%, seed = shape index."""
    return synth.make_layer(*SHAPES[name], bits=4, group_size=128, rank=16, density=0.005, seed=NAMES.index(name))


@functools.lru_cache(maxsize=None)
def merged(name: str) -> synth.SynthLayer:
    parts = {"qkv_proj": ["q_proj", "k_proj", "v_proj"], "gate_up_proj": ["gate_proj", "up_proj"]}.get(name, [name])
    if len(parts) == 1:
        return unmerged(parts[0])
    return synth.merge_layers([unmerged(p) for p in parts])


def _decode(vw, L: synth.SynthLayer, label: str):
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, L.bits, L.group_size, t["chunk_offsets"],
                               t["chunk_cols"], t["chunk_vals"])
    assert prep.numel() > 0, "the 7B layers have a prepared layout"
    rows = pick_rows(L, 224, seed=L.N)
    for M in (1, 4, 8, 16, 32):
        _case(f"decode {label} {L.N}x{L.K} r={L.rank} M={M}")
        x = synth.make_activations(M, L.K, seed=1000 + M)
        y, H = run_prepared(vw, L, x, dora="fused", prep=prep, t=t)
        assert np.all(np.isfinite(y.astype(np.float32))), f"{label} M={M}: non-finite output"
        check_rows(y[:, rows], x, L, rows, H, what=f"{label} M={M}", reference_rounding=M >= 16)
    del t, prep
    torch.cuda.empty_cache()


@pytest.mark.parametrize("name", ["qkv_proj", "o_proj", "gate_up_proj", "down_proj"])
def test_decode_merged_7b(vw, name):
    """vLLM's merged projections through the prepared decode kernel (the benchmark's step)."""
    _decode(vw, merged(name), name)


@pytest.mark.parametrize("name", NAMES)
def test_decode_unmerged_7b(vw, name):
    """The seven projections one by one (the benchmark's per-shape figures)."""
    _decode(vw, unmerged(name), name)


@pytest.mark.parametrize("name", NAMES)
def test_prefill_7b(vw, name):
    """Config 2: M = 128, 512, 2048, 8192 through the op as apply() issues it (prepared
    buffer passed, lora_A given so H = fp16(X A^T) is computed on the device).  24
    activation rows (both ends, both sides of the 256-row tile edges, random) x the
    checked output rows."""
    L = unmerged(name)
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, L.bits, L.group_size, t["chunk_offsets"],
                               t["chunk_cols"], t["chunk_vals"])
    rows = pick_rows(L, 160, seed=7 * L.N)
    for M in (128, 512, 2048, 8192):
        _case(f"prefill {name} {L.N}x{L.K} M={M}")
        gen = torch.Generator(device=DEV)
        gen.manual_seed(M + L.N)
        X = torch.randn(M, L.K, generator=gen, device=DEV).half()
        out = torch.empty(M, L.N, dtype=torch.float16, device=DEV)
        torch.ops.wlq_fastShot.gemm(X, t["q_packed"], t["lut_c"], out, L.N, L.K, L.bits, L.wpr, t["chunk_offsets"],
                                    t["chunk_cols"], t["chunk_vals"], None, t["lora_B"], t["dora_gamma"],
                                    L.lora_scale, L.group_size, t["lora_A"], prep)
        torch.cuda.synchronize()
        rng = np.random.default_rng(M)
        xr = {0, M - 1}
        xr |= {min(M - 1, v) for v in (127, 128, 255, 256, 511, 512)}
        xr |= set(rng.choice(M, size=16, replace=False).tolist())
        xr = np.array(sorted(xr))
        # host-side bounds check before the device gathers (index_select does not check on the device)
        assert xr.min() >= 0 and xr.max() < M and rows.min() >= 0 and rows.max() < L.N
        xr_t = torch.from_numpy(xr).to(DEV)
        rows_t = torch.from_numpy(rows).to(DEV)
        y = out.index_select(0, xr_t).index_select(1, rows_t).cpu().numpy()
        x = X.index_select(0, xr_t).cpu().numpy()
        assert bool(torch.isfinite(out).all()), f"{name} M={M}: non-finite output"
        H = O.lora_h(x, L.A)
        check_rows(y, x, L, rows, H, what=f"{name} M={M}", reference_rounding=True)
        del X, out
    del t, prep
    torch.cuda.empty_cache()
