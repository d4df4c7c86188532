"""GPU parity of the M = 9..128 product on the prepared layout (wlq_wide.hip) against the
CPU oracle: M on both sides of the 16-row MFMA groups and of the 16 / 32 / 64 / 128
activation buffers, LUT per row / per lane segment / per slab / general groups, DoRA H
computed in the kernel / given / off, outliers on and off (incl. blocks of 16 x 128
weights with more patches than the kernel's LDS list holds), 3-bit layers, K splits,
ragged N and K, back-to-back calls of different M on one workspace, graph replay and
determinism.  Tolerance: gpu_helpers.REL_TOL against the single-rounding oracle and,
as the reference rounds x.W0^T to fp16 first from M = 16 (csrc/vllm_binding.cpp:355-393),
against that rounding as well."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, check_close, oracle_product, run_prepared
from qwen_wlqfastshot_helen_beta_amd import synth

pytestmark = pytest.mark.gpu

MS = [9, 16, 17, 32, 33, 48, 64, 65, 100, 128]


def _case(**kw):
    print("[case] " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _check(y, L, x, H, what, with_csr=True):
    check_close(y, oracle_product(L, x, H, with_csr=with_csr), what=what)
    if x.shape[0] >= 16:
        check_close(y, oracle_product(L, x, H, with_csr=with_csr, round_gemm_output=None), what=what + " ref-rounding")


@pytest.mark.parametrize("M", MS)
def test_wide_parity(vw, M):
    for gs in (0, 64, 128, 384):
        for dora in ("fused", "h", "none"):
            _case(M=M, gs=gs, dora=dora)
            L = synth.make_layer(N=200, K=1408, bits=4, group_size=gs, rank=8, density=0.01, seed=500 + M + gs)
            x = synth.make_activations(M, L.K, seed=M + 1)
            y, H = run_prepared(vw, L, x, dora=dora)
            _check(y, L, x, H, f"M={M} gs={gs} dora={dora}")


@pytest.mark.parametrize("M", [9, 64, 128])
def test_wide_without_outliers(vw, M):
    _case(M=M, csr=False)
    L = synth.make_layer(N=136, K=1024, bits=4, group_size=128, rank=16, density=0.01, seed=M)
    x = synth.make_activations(M, L.K, seed=7 * M)
    y, H = run_prepared(vw, L, x, dora="fused", with_csr=False)
    _check(y, L, x, H, f"M={M} no csr", with_csr=False)


@pytest.mark.parametrize("M", [12, 32, 65, 128])
def test_wide_3bit(vw, M):
    """3-bit: codes widened to nibbles against 8-entry LUTs, 640-column outlier chunks."""
    for gs in (0, 128):
        _case(M=M, gs=gs, bits=3)
        L = synth.make_layer(N=150, K=1928, bits=3, group_size=gs, rank=8, density=0.01, seed=900 + M + gs)
        x = synth.make_activations(M, L.K, seed=M)
        y, H = run_prepared(vw, L, x, dora="fused")
        _check(y, L, x, H, f"3-bit M={M} gs={gs}")


@pytest.mark.parametrize("M", [16, 128])
def test_wide_dense_outliers(vw, M):
    """20% outliers: ~410 patches per 16 x 128 block, beyond the 256 the LDS list holds, so
    the rest are applied from global memory."""
    _case(M=M, density=0.2)
    L = synth.make_layer(N=64, K=1024, bits=4, group_size=128, rank=8, density=0.2, seed=M)
    x = synth.make_activations(M, L.K, seed=M)
    y, H = run_prepared(vw, L, x, dora="h")
    _check(y, L, x, H, f"dense outliers M={M}")


@pytest.mark.parametrize("rank", [16, 48, 64])
def test_wide_ranks(vw, rank):
    for M in (33, 128):
        for dora in ("fused", "h"):
            _case(M=M, rank=rank, dora=dora)
            L = synth.make_layer(N=256, K=2048, bits=4, group_size=128, rank=rank, density=0.005, seed=rank + M)
            x = synth.make_activations(M, L.K, seed=rank)
            y, H = run_prepared(vw, L, x, dora=dora)
            _check(y, L, x, H, f"rank={rank} M={M} dora={dora}")


@pytest.mark.parametrize("shape", [(100, 18944), (48, 8192), (4864, 896), (20, 1928)])
def test_wide_splits_and_shapes(vw, shape):
    """K = 18944 has 148 slabs (more than one split holds); few row tiles split K many ways;
    K = 1928 ends in a partial slab."""
    N, K = shape
    for M in (9, 64, 128):
        _case(N=N, K=K, M=M)
        L = synth.make_layer(N=N, K=K, bits=4, group_size=128, rank=16, density=0.005, seed=N + M)
        x = synth.make_activations(M, K, seed=M)
        y, H = run_prepared(vw, L, x, dora="fused")
        _check(y, L, x, H, f"{N}x{K} M={M}")


def test_wide_back_to_back(vw):
    """Calls of different M in a row on one stream's workspace: each leaves the counters
    and ready slots as the next expects."""
    L = synth.make_layer(N=300, K=4096, bits=4, group_size=128, rank=16, density=0.005, seed=3)
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, L.bits, L.group_size, t["chunk_offsets"],
                               t["chunk_cols"], t["chunk_vals"])
    for M in (128, 9, 64, 33, 128, 16):
        _case(M=M, seq=True)
        x = synth.make_activations(M, L.K, seed=M + 50)
        y, H = run_prepared(vw, L, x, dora="fused", prep=prep, t=t)
        _check(y, L, x, H, f"sequence M={M}")
    vw.check_workspaces(DEV)  # raises if a hand-off failed


def test_wide_deterministic_and_graph_replay(vw):
    """Same inputs give the same bits; a captured call replays to the eager result, with
    eager work of other shapes between the replays."""
    L = synth.make_layer(N=512, K=3584, bits=4, group_size=128, rank=16, density=0.005, seed=11)
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, L.bits, L.group_size, t["chunk_offsets"],
                               t["chunk_cols"], t["chunk_vals"])
    M = 64
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
    x2 = torch.from_numpy(synth.make_activations(17, L.K, seed=2)).to(DEV)
    o2 = torch.empty(17, L.N, dtype=torch.float16, device=DEV)
    for rep in range(3):
        _case(replay=rep)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
        call(x2, o2)  # eager work between replays
        torch.cuda.synchronize()
    vw.check_workspaces(DEV)  # raises if a hand-off failed


def test_wide_kernel_is_the_one_that_runs(vw):
    """The M = 9..128 calls run the wide kernel (kernel names from the profiler)."""
    L = synth.make_layer(N=256, K=1024, bits=4, group_size=128, rank=8, density=0.01, seed=4)
    x = synth.make_activations(64, L.K, seed=4)
    run_prepared(vw, L, x, dora="fused")  # warm-up
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        run_prepared(vw, L, x, dora="fused")
        torch.cuda.synchronize()
    names = [e.name for e in prof.events()]
    if not any("wlq" in n for n in names):
        pytest.skip("the profiler recorded no kernels of the library")
    assert any("wide_kernel" in n for n in names), sorted(set(names))


@pytest.mark.parametrize("scale", [0.37, 3e5])
def test_wide_given_h_fp32(vw, scale):
    """A caller's fp32 H (the op's lora_H, fp32 as the reference takes it,
    csrc/gemm_kernel.cu:449-466): values that are not fp16 numbers, and (3e5) values beyond the
    fp16 range, which the kernel scales by a power of two before its fp16 MFMA parts."""
    L = synth.make_layer(N=192, K=1024, bits=4, group_size=128, rank=16, density=0.01, seed=21)
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, L.bits, L.group_size, t["chunk_offsets"],
                               t["chunk_cols"], t["chunk_vals"])
    for M in (20, 100):
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


@pytest.mark.parametrize("M", [65, 128])
def test_wide_two_tiles_per_wave(vw, M):
    """128-row activation buffers on a layer long in K (65 slabs) run two 16-row W tiles per
    compute wave (128-row blocks); N = 136 leaves the second block with one tile.  Every LUT
    mode, DoRA fused / given / off, 3-bit, and 20% outliers (lists beyond the LDS list)."""
    cases = [(4, gs, dora, 0.01) for gs in (0, 64, 128, 384) for dora in ("fused", "h", "none")]
    cases += [(3, 128, "fused", 0.01), (4, 128, "fused", 0.2)]
    for bits, gs, dora, d in cases:
        _case(M=M, bits=bits, gs=gs, dora=dora, density=d)
        L = synth.make_layer(N=136, K=8320, bits=bits, group_size=gs, rank=16, density=d, seed=M + gs + bits)
        x = synth.make_activations(M, L.K, seed=M + 3)
        y, H = run_prepared(vw, L, x, dora=dora)
        _check(y, L, x, H, f"two tiles M={M} bits={bits} gs={gs} dora={dora} d={d}")
