"""GPU parity of the prefill GEMM (wlq_gemm.hip) on a prepared layer: outliers taken from the
prepared buffer's patch lists (per 16-row tile and 128-column slab) instead of per-call records,
against the CPU oracle.  Cases: ragged N (N tiles of 128 rows with missing 16-row tiles) and K
(partial chunks and slabs), per-row LUTs and LUT groups of 64 / 128 / 256 columns, 3-bit layers
(640-column chunks: five slabs per chunk), K splits (list starts of a block's range that do not
begin at slab 0), dense outliers (lists longer than the 32 entries a list's threads take per
slab: those waves walk their rows' CSR entries) and heavy rows (waves of both kinds in one
block), prepared layers without outliers, DoRA H computed / given / off.  Tolerance: gpu_helpers.REL_TOL against the
single-rounding oracle and against the reference's fp16 rounding of x.W0^T
(csrc/vllm_binding.cpp:355-393)."""
from __future__ import annotations

import pytest
import torch

from gpu_helpers import check_close, oracle_product, run_prepared
from qwen_wlqfastshot_helen_beta_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _no_forced_prefill(monkeypatch):
    """These shapes are narrow enough that the library picks the GEMM for M > 128."""
    monkeypatch.delenv("WLQ_TEST_FORCE_PREFILL", raising=False)


def _case(**kw):
    print("[case] " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _check(y, L, x, H, what):
    check_close(y, oracle_product(L, x, H), what=what)
    check_close(y, oracle_product(L, x, H, round_gemm_output=None), what=what + " ref-rounding")


@pytest.mark.parametrize("M", [129, 200, 300, 520])
def test_gemm_lists_parity(vw, M):
    for N, gs in ((200, 128), (1000, 0), (200, 64), (1000, 256)):
        for dora in ("fused", "h", "none"):
            if dora != "fused" and N == 1000:
                continue
            _case(M=M, N=N, gs=gs, dora=dora)
            L = synth.make_layer(N=N, K=1408, bits=4, group_size=gs, rank=8, density=0.01, seed=M + N + gs)
            x = synth.make_activations(M, L.K, seed=M + 3)
            y, H = run_prepared(vw, L, x, dora=dora)
            _check(y, L, x, H, f"M={M} N={N} gs={gs} dora={dora}")


@pytest.mark.parametrize("M", [150, 400])
def test_gemm_lists_3bit(vw, M):
    for gs in (0, 128):
        _case(M=M, gs=gs, bits=3)
        L = synth.make_layer(N=270, K=1928, bits=3, group_size=gs, rank=8, density=0.01, seed=40 + M + gs)
        x = synth.make_activations(M, L.K, seed=M)
        y, H = run_prepared(vw, L, x, dora="fused")
        _check(y, L, x, H, f"3-bit M={M} gs={gs}")


@pytest.mark.parametrize("shape", [(256, 8192), (100, 18944), (40, 3000)])
def test_gemm_lists_splits(vw, shape):
    """Few N tiles: K is split over blocks, each reading the list starts of its own slabs."""
    N, K = shape
    for M in (129, 256):
        _case(N=N, K=K, M=M)
        L = synth.make_layer(N=N, K=K, bits=4, group_size=128, rank=16, density=0.005, seed=N + M)
        x = synth.make_activations(M, K, seed=M + 9)
        y, H = run_prepared(vw, L, x, dora="fused")
        _check(y, L, x, H, f"{N}x{K} M={M}")


@pytest.mark.parametrize("density,heavy", [(0.2, 0.0), (0.02, 0.2)])
def test_gemm_lists_long(vw, density, heavy):
    """20% outliers: ~400 per list and slab, every wave walks the CSR entries; 2% with 20% heavy
    rows (10x the mean): lists beyond 32 entries in some waves only."""
    for M in (130, 300):
        _case(M=M, density=density, heavy=heavy)
        L = synth.make_layer(N=384, K=1024, bits=4, group_size=128, rank=8, density=density, heavy_frac=heavy,
                             seed=int(density * 1000) + M)
        x = synth.make_activations(M, L.K, seed=M)
        y, H = run_prepared(vw, L, x, dora="h")
        _check(y, L, x, H, f"density={density} heavy={heavy} M={M}")


def test_gemm_lists_kernels(vw):
    """A prepared layer's GEMM takes its outliers from the prepared lists: no per-call outlier
    records are built."""
    L = synth.make_layer(N=512, K=2048, bits=4, group_size=128, rank=8, density=0.01, seed=5)
    x = synth.make_activations(300, L.K, seed=5)
    run_prepared(vw, L, x, dora="fused")  # warm-up
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        run_prepared(vw, L, x, dora="fused")
        torch.cuda.synchronize()
    names = [e.name for e in prof.events()]
    if not any("wlq" in n for n in names):
        pytest.skip("the profiler recorded no kernels of the library")
    assert any("gemm_kernel" in n for n in names), sorted(set(names))
    assert not any("tile_entries_kernel" in n for n in names), sorted(set(names))


@pytest.mark.parametrize("rank", [8, 24, 48, 64, 80])
def test_gemm_dora_ranks(vw, rank):
    """The GEMM's DoRA epilogue reads H, B rows and gamma staged in LDS by the producer waves:
    up to 16 ranks loaded during the last K step, more in rounds of 64 (80: two rounds, the
    second partial), H computed by the library or given by the caller."""
    for M, dora in ((200, "fused"), (300, "h")):
        _case(M=M, rank=rank, dora=dora)
        L = synth.make_layer(N=300, K=1408, bits=4, group_size=128, rank=rank, density=0.01, seed=rank + M)
        x = synth.make_activations(M, L.K, seed=rank)
        y, H = run_prepared(vw, L, x, dora=dora)
        _check(y, L, x, H, f"rank={rank} M={M} dora={dora}")


@pytest.mark.parametrize("bits", [4, 3])
def test_gemm_prepared_codes_no_outliers(vw, bits):
    """A prepared layer without outliers: the GEMM reads the prepared codes and LUT planes (3-bit
    layers as nibbles with 16-entry planes) and applies no patches."""
    for M, gs in ((150, 0), (300, 128), (260, 64)):
        _case(M=M, gs=gs, bits=bits, csr=False)
        L = synth.make_layer(N=330, K=1408 if bits == 4 else 1928, bits=bits, group_size=gs, rank=16, density=0.01,
                             seed=bits * 100 + M + gs)
        x = synth.make_activations(M, L.K, seed=M + gs)
        y, H = run_prepared(vw, L, x, dora="fused", with_csr=False)
        check_close(y, oracle_product(L, x, H, with_csr=False), what=f"no csr bits={bits} M={M} gs={gs}")
