"""Config 3 (outlier / adapter stress) at the full gate_proj shape 18944 x 3584:
outlier density 0.1-2% with 20% heavy rows holding 10x the mean, DoRA rank 0/8/16/64,
LUT groups 64 and 128, 4-bit and 3-bit, M = 1, 4 and 512.  The oracle checks a
random subset of output rows (sliced out of the layer with their CSR entries), which
keeps the CPU side to seconds at the full shape.  Each case runs both the row-aligned
kernel and the prepared-layout path that a loaded layer uses."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_helpers import check_rows, pick_rows, run_prepared, run_product
from qwen_wlqfastshot_helen_beta_amd import synth

pytestmark = pytest.mark.gpu

GATE = synth.QWEN25_7B_SHAPES["gate_proj"]


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _check(vw, L, M, seed, what):
    """Row-layout kernel (no prepared buffer) and the prepared path apply() uses, both
    against the oracle on a row subset that includes the densest (heavy) rows."""
    x = synth.make_activations(M, L.K, seed=seed)
    rows = pick_rows(L, 192, seed=seed, heavy=64)
    y, H = run_product(vw, L, x, fused_h=L.B is not None)
    check_rows(y[:, rows], x, L, rows, H, what=what + " row layout", reference_rounding=M >= 16)
    yp, Hp = run_prepared(vw, L, x, dora="fused" if L.B is not None else "none")
    check_rows(yp[:, rows], x, L, rows, Hp, what=what + " prepared", reference_rounding=M >= 16)


@pytest.mark.parametrize("density", [0.001, 0.005, 0.01, 0.02])
def test_gate_outlier_density_heavy_rows(vw, density):
    _case(f"gate density={density} heavy 20%x10 r=16 G=128 M=1,4")
    L = synth.make_layer(*GATE, bits=4, group_size=128, rank=16, density=density, seed=31, heavy_frac=0.2,
                         heavy_mult=10.0)
    for M in (1, 4):
        _check(vw, L, M, seed=M, what=f"d={density} M={M}")


@pytest.mark.parametrize("rank,gs", [(0, 64), (8, 64), (64, 128)])
def test_gate_rank_and_group(vw, rank, gs):
    _case(f"gate rank={rank} G={gs} M=1")
    L = synth.make_layer(*GATE, bits=4, group_size=gs, rank=rank, density=0.005, seed=32, heavy_frac=0.2,
                         heavy_mult=10.0)
    _check(vw, L, 1, seed=5, what=f"r={rank} G={gs}")


def test_gate_3bit(vw):
    _case("gate 3-bit G=128 M=1")
    L = synth.make_layer(*GATE, bits=3, group_size=128, rank=16, density=0.01, seed=33, heavy_frac=0.2,
                         heavy_mult=10.0)
    _check(vw, L, 1, seed=6, what="3-bit")


def test_gate_prefill_m512(vw):
    _case("gate M=512 d=2% heavy r=16 G=64")
    L = synth.make_layer(*GATE, bits=4, group_size=64, rank=16, density=0.02, seed=34, heavy_frac=0.2,
                         heavy_mult=10.0)
    _check(vw, L, 512, seed=7, what="M=512")
