"""GPU parity of the M > 128 product on the prepared layout (wlq_prefill.hip, 32x32x16 MFMA
with W dequantized in registers) against the CPU oracle: M on both sides of the 32-row MFMA
groups and of the 128-row activation blocks, ragged N (blocks of 256 W rows) and K (partial
slabs), per-row LUTs and LUT groups of 128 / 256 columns (groups of 64 or 384 columns take the
MFMA GEMM and are covered there), DoRA H computed in the kernel / given / off at ranks 8..64,
outliers on and off (incl. lists longer than the 64 patches a lane set applies per slab),
3-bit layers, K splits (layers longer than one split holds), back-to-back calls of different M on
one workspace,
graph replay and determinism.  Tolerance: gpu_helpers.REL_TOL against the single-rounding
oracle and against the reference's fp16 rounding of x.W0^T (csrc/vllm_binding.cpp:355-393)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, check_close, oracle_product, run_prepared
from qwen_wlqfastshot_helen_beta_amd import synth

pytestmark = pytest.mark.gpu

MS = [129, 160, 255, 256, 300, 512]


@pytest.fixture(autouse=True)
def _force_prefill(monkeypatch):
    """The library takes this kernel by itself only where it measured faster than the MFMA GEMM
    (wide layers, K <= 4096); the test hook makes it run these small shapes too."""
    monkeypatch.setenv("WLQ_TEST_FORCE_PREFILL", "1")


def _case(**kw):
    print("[case] " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _check(y, L, x, H, what, with_csr=True):
    check_close(y, oracle_product(L, x, H, with_csr=with_csr), what=what)
    check_close(y, oracle_product(L, x, H, with_csr=with_csr, round_gemm_output=None), what=what + " ref-rounding")


@pytest.mark.parametrize("M", MS)
def test_prefill_parity(vw, M):
    for gs in (0, 128, 256):
        for dora in ("fused", "h", "none"):
            _case(M=M, gs=gs, dora=dora)
            L = synth.make_layer(N=300, K=1408, bits=4, group_size=gs, rank=8, density=0.01, seed=700 + M + gs)
            x = synth.make_activations(M, L.K, seed=M + 1)
            y, H = run_prepared(vw, L, x, dora=dora)
            _check(y, L, x, H, f"M={M} gs={gs} dora={dora}")


@pytest.mark.parametrize("M", [129, 384])
def test_prefill_without_outliers(vw, M):
    _case(M=M, csr=False)
    L = synth.make_layer(N=520, K=1024, bits=4, group_size=128, rank=16, density=0.01, seed=M)
    x = synth.make_activations(M, L.K, seed=7 * M)
    y, H = run_prepared(vw, L, x, dora="fused", with_csr=False)
    _check(y, L, x, H, f"M={M} no csr", with_csr=False)


@pytest.mark.parametrize("M", [200, 512])
def test_prefill_3bit(vw, M):
    """3-bit: codes widened to nibbles against 8-entry LUTs, 640-column outlier chunks."""
    for gs in (0, 128):
        _case(M=M, gs=gs, bits=3)
        L = synth.make_layer(N=270, K=1928, bits=3, group_size=gs, rank=8, density=0.01, seed=900 + M + gs)
        x = synth.make_activations(M, L.K, seed=M)
        y, H = run_prepared(vw, L, x, dora="fused")
        _check(y, L, x, H, f"3-bit M={M} gs={gs}")


@pytest.mark.parametrize("M", [129, 256])
def test_prefill_dense_outliers(vw, M):
    """20% outliers: ~410 patches per 16 x 128 block, beyond the 64 the lanes apply from
    registers, so the rest are applied from global memory."""
    _case(M=M, density=0.2)
    L = synth.make_layer(N=256, K=1024, bits=4, group_size=128, rank=8, density=0.2, seed=M)
    x = synth.make_activations(M, L.K, seed=M)
    y, H = run_prepared(vw, L, x, dora="h")
    _check(y, L, x, H, f"dense outliers M={M}")


@pytest.mark.parametrize("rank", [16, 48, 64])
def test_prefill_ranks(vw, rank):
    for M in (130, 256):
        for dora in ("fused", "h"):
            _case(M=M, rank=rank, dora=dora)
            L = synth.make_layer(N=512, K=2048, bits=4, group_size=128, rank=rank, density=0.005, seed=rank + M)
            x = synth.make_activations(M, L.K, seed=rank)
            y, H = run_prepared(vw, L, x, dora=dora)
            _check(y, L, x, H, f"rank={rank} M={M} dora={dora}")


@pytest.mark.parametrize("shape", [(100, 18944), (512, 3584), (4864, 896), (40, 1928), (300, 26000)])
def test_prefill_splits_and_shapes(vw, shape):
    """K = 18944: 148 slabs in one split (within the 191 a split holds); K = 26000: 204
    slabs, two splits and the split-order sum; N = 40 and 100 leave most of a 256-row block
    empty; K = 1928 ends in a partial slab."""
    N, K = shape
    for M in (129, 256):
        _case(N=N, K=K, M=M)
        L = synth.make_layer(N=N, K=K, bits=4, group_size=128, rank=16, density=0.005, seed=N + M)
        x = synth.make_activations(M, K, seed=M)
        y, H = run_prepared(vw, L, x, dora="fused")
        _check(y, L, x, H, f"{N}x{K} M={M}")


def test_prefill_back_to_back(vw):
    """Calls of different M in a row on one stream's workspace (prefill, decode and wide
    kernels): each leaves the counters and ready slots as the next expects."""
    L = synth.make_layer(N=300, K=4096, bits=4, group_size=128, rank=16, density=0.005, seed=3)
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, L.bits, L.group_size, t["chunk_offsets"],
                               t["chunk_cols"], t["chunk_vals"])
    for M in (256, 129, 1, 600, 64, 384, 130):
        _case(M=M, seq=True)
        x = synth.make_activations(M, L.K, seed=M + 50)
        y, H = run_prepared(vw, L, x, dora="fused", prep=prep, t=t)
        _check(y, L, x, H, f"sequence M={M}")
    vw.check_workspaces(DEV)  # raises if a hand-off failed


def test_prefill_deterministic_and_graph_replay(vw):
    """Same inputs give the same bits; a captured call replays to the eager result, with
    eager work of other shapes between the replays."""
    L = synth.make_layer(N=512, K=3584, bits=4, group_size=128, rank=16, density=0.005, seed=11)
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, L.bits, L.group_size, t["chunk_offsets"],
                               t["chunk_cols"], t["chunk_vals"])
    M = 384
    x = torch.from_numpy(synth.make_activations(M, L.K, seed=1)).to(DEV)
    out = torch.empty(M, L.N, dtype=torch.float16, device=DEV)

    def call(xx, oo):
        torch.ops.wlq_fastShot.gemm(xx, t["q_packed"], t["lut_c"], oo, L.N, L.K, L.bits, L.wpr, t["chunk_offsets"],
                                    t["chunk_cols"], t["chunk_vals"], None, t["lora_B"], t["dora_gamma"],
                                    L.lora_scale, L.group_size, t["lora_A"], prep)

    call(x, out)
    torch.cuda.synchronize()
    eager = out.clone()
    call(x, out)
    torch.cuda.synchronize()
    assert torch.equal(out, eager), "not deterministic"
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call(x, out)  # warm-up on the capture stream (its workspace)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(x, out)
    x2 = torch.from_numpy(synth.make_activations(200, L.K, seed=2)).to(DEV)
    o2 = torch.empty(200, L.N, dtype=torch.float16, device=DEV)
    for rep in range(3):
        _case(replay=rep)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
        call(x2, o2)  # eager work between replays
        torch.cuda.synchronize()
    vw.check_workspaces(DEV)


def test_prefill_kernel_is_the_one_that_runs(vw):
    """M > 128 calls on a prepared layer with slab-aligned LUT groups run the prefill kernel."""
    L = synth.make_layer(N=256, K=1024, bits=4, group_size=128, rank=8, density=0.01, seed=4)
    x = synth.make_activations(256, L.K, seed=4)
    run_prepared(vw, L, x, dora="fused")  # warm-up
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        run_prepared(vw, L, x, dora="fused")
        torch.cuda.synchronize()
    names = [e.name for e in prof.events()]
    if not any("wlq" in n for n in names):
        pytest.skip("the profiler recorded no kernels of the library")
    assert any("prefill_kernel" in n for n in names), sorted(set(names))


@pytest.mark.parametrize("scale", [0.37, 3e5])
def test_prefill_given_h_fp32(vw, scale):
    """A caller's fp32 H: values that are not fp16 numbers, and (3e5) values beyond the fp16
    range, which the kernel scales by a power of two before its fp16 MFMA parts."""
    L = synth.make_layer(N=320, K=1024, bits=4, group_size=128, rank=16, density=0.01, seed=21)
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, L.bits, L.group_size, t["chunk_offsets"],
                               t["chunk_cols"], t["chunk_vals"])
    for M in (140, 300):
        _case(M=M, h_scale=scale)
        x = synth.make_activations(M, L.K, seed=M)
        H = (np.random.default_rng(M).standard_normal((M, L.rank)) * scale).astype(np.float32)
        out = torch.empty(M, L.N, dtype=torch.float16, device=DEV)
        torch.ops.wlq_fastShot.gemm(torch.from_numpy(x).to(DEV), t["q_packed"], t["lut_c"], out, L.N, L.K, L.bits,
                                    L.wpr, t["chunk_offsets"], t["chunk_cols"], t["chunk_vals"],
                                    torch.from_numpy(H).to(DEV), t["lora_B"], t["dora_gamma"], L.lora_scale,
                                    L.group_size, None, prep)
        torch.cuda.synchronize()
        y = out.cpu().numpy()
        ref = oracle_product(L, x, H)
        if scale > 1e4:  # outputs beyond fp16 become inf in both; compare the finite ones
            fin = np.isfinite(ref.astype(np.float64)) & (np.abs(ref.astype(np.float64)) < 6e4)
            assert fin.mean() > 0.2
            yy, rr = y.astype(np.float64)[fin], ref.astype(np.float64)[fin]
            assert np.max(np.abs(yy - rr)) <= 2e-3 * np.max(np.abs(rr)) + 1e-6, f"M={M} scale={scale}"
        else:
            check_close(y, ref, what=f"given fp32 H M={M}")
