"""GPU parity of the prepared-layout products (wlq_stream.hip for M <= 8, wlq_wide.hip
for M = 9..128) against the CPU oracle: the prepared layout itself bit-exact against a numpy rebuild, layer
outputs within the tolerance of tests/gpu_helpers.py, across M = 1..32, LUT
group sizes, ragged shapes, outliers on/off (incl. heavy rows), DoRA fused / H
given / off, split-K, counter reset between calls, graph replay, determinism,
and the C ABI entry point."""
import numpy as np
import pytest
import torch

from gpu_helpers import (DEV, check_close, oracle_product, prepared_reference, run_prepared, run_product,
                         split_prepared, wide_patches_reference)
from qwen_wlqfastshot_helen_beta_amd import synth

pytestmark = pytest.mark.gpu


def _case(**kw):
    print("[case] " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@pytest.mark.parametrize("bits,gs", [(4, 0), (4, 32), (4, 64), (4, 128), (4, 256), (3, 0), (3, 64), (3, 128)])
def test_prepared_layout_bit_exact(vw, bits, gs):
    for N, K, density in ((77, 1000, 0.02), (64, 512, 0.0), (33, 3584, 0.005), (20, 1928, 0.03)):
        _case(bits=bits, gs=gs, N=N, K=K, density=density)
        L = synth.make_layer(N=N, K=K, bits=bits, group_size=gs, rank=0, density=density, seed=N + gs)
        t = L.to_torch(DEV)
        buf = vw._C.prepare_layer(t["q_packed"], t["lut_c"], N, K, bits, gs, t["chunk_offsets"], t["chunk_cols"],
                                  t["chunk_vals"])
        torch.cuda.synchronize()
        assert buf.numel() > 0
        got = split_prepared(buf.cpu().numpy(), L)
        ref = prepared_reference(L)
        assert np.array_equal(got[0], ref[0]), "codes"
        assert np.array_equal(got[1], ref[1]), "planes"
        assert np.array_equal(got[2].astype(np.int64), ref[2]), "gcol"
        assert np.array_equal(got[3].view(np.uint32), ref[3].view(np.uint32)), "delta"
        if L.nnz > 0:
            wpidx, wpatch = wide_patches_reference(N, K, bits, L.offsets, L.cols, L.vals)
            assert np.array_equal(got[4], wpidx), "patch-list starts"
            assert np.array_equal(got[5][:wpatch.size], wpatch), "patches"


def test_prepare_unsupported_formats(vw):
    """2- and 1-bit codes, group sizes not a multiple of 32 and K % 8 != 0 have no prepared layout."""
    for bits, gs, K in ((2, 64, 640), (1, 128, 1024), (4, 48, 960), (3, 48, 960), (4, 128, 1001)):
        L = synth.make_layer(N=16, K=K, bits=bits, group_size=gs, rank=0, density=0.0, seed=1)
        t = L.to_torch(DEV)
        buf = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, bits, gs)
        assert buf.numel() == 0, (bits, gs, K)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 9, 13, 16, 17, 24, 32])
def test_prepared_parity(vw, M):
    """M <= 16: one MFMA row group; 17..32: two (rows 16..31 share the dequantized W).
    From M = 16 the reference rounds the GEMM output to fp16 before the DoRA epilogue
    (csrc/vllm_binding.cpp:355-393); the single rounding here is within tolerance of both."""
    for gs in (0, 32, 64, 128, 256, 384):  # per row; groups per lane segment; per slab (128 << k); general
        for dora in ("fused", "h", "none"):
            _case(M=M, gs=gs, dora=dora)
            L = synth.make_layer(N=200, K=1408, bits=4, group_size=gs, rank=8, density=0.01, seed=100 + M + gs)
            x = synth.make_activations(M, L.K, seed=M)
            y, H = run_prepared(vw, L, x, dora=dora)
            check_close(y, oracle_product(L, x, H), what=f"M={M} gs={gs} dora={dora}")
            if M >= 16:
                check_close(y, oracle_product(L, x, H, round_gemm_output=None), what=f"M={M} reference rounding")


@pytest.mark.parametrize("M", [1, 2, 4, 8, 12, 13, 16, 17, 25, 26, 32])
def test_prepared_parity_3bit(vw, M):
    """3-bit layers: codes widened to nibbles, 640-column outlier chunks (5 slabs); M <= 8
    on the decode kernel, M >= 9 on the M = 9..128 kernel."""
    for gs in (0, 64, 128):
        for dora in ("fused", "h"):
            _case(M=M, gs=gs, dora=dora, bits=3)
            L = synth.make_layer(N=200, K=1928, bits=3, group_size=gs, rank=8, density=0.01, seed=300 + M + gs)
            x = synth.make_activations(M, L.K, seed=M)
            y, H = run_prepared(vw, L, x, dora=dora)
            check_close(y, oracle_product(L, x, H), what=f"3-bit M={M} gs={gs} dora={dora}")


@pytest.mark.parametrize("shape", [(48, 8192), (16, 3584), (4864, 896), (100, 18944), (512, 3584)])
def test_prepared_shapes_and_splits(vw, shape):
    """Narrow layers (many K splits), config-0 up_proj, a down_proj-like K."""
    N, K = shape
    for M in (1, 4, 32):
        _case(N=N, K=K, M=M)
        L = synth.make_layer(N=N, K=K, bits=4, group_size=128, rank=16, density=0.005, seed=N + K + M)
        x = synth.make_activations(M, L.K, seed=M + 7)
        y, H = run_prepared(vw, L, x, dora="fused")
        check_close(y, oracle_product(L, x, H), what=f"N={N} K={K} M={M}")


@pytest.mark.parametrize("shape", [(48, 8960), (4864, 896), (100, 18944), (3000, 3584)])
def test_prepared_shapes_3bit(vw, shape):
    N, K = shape
    for M in (1, 4, 8):
        _case(N=N, K=K, M=M, bits=3)
        L = synth.make_layer(N=N, K=K, bits=3, group_size=64, rank=16, density=0.005, seed=N + K + M)
        x = synth.make_activations(M, L.K, seed=M + 7)
        y, H = run_prepared(vw, L, x, dora="fused")
        check_close(y, oracle_product(L, x, H), what=f"3-bit N={N} K={K} M={M}")
        b, _ = run_product(vw, L, x, fused_h=True)
        check_close(y, b.astype(np.float64), tol=1.2e-3, what=f"3-bit prepared vs row layout N={N} K={K} M={M}")


@pytest.mark.parametrize("shape", [(4112, 1024), (4864, 896), (8208, 3584)])
def test_prepared_two_tiles_per_block(vw, shape):
    """M <= 2 on layers with >= 256 row tiles: blocks of two 16-row tiles (an odd tile count
    leaves the last block's second tile past N)."""
    N, K = shape
    for M in (1, 2):
        for gs, dora in ((128, "fused"), (0, "h"), (64, "none")):
            _case(N=N, K=K, M=M, gs=gs, dora=dora)
            L = synth.make_layer(N=N, K=K, bits=4, group_size=gs, rank=16, density=0.01, seed=N + M + gs)
            x = synth.make_activations(M, L.K, seed=M + 3)
            y, H = run_prepared(vw, L, x, dora=dora)
            check_close(y, oracle_product(L, x, H), what=f"N={N} K={K} M={M} gs={gs} dora={dora}")


def test_prepared_no_outliers_and_heavy_rows(vw):
    for M in (1, 4, 8):
        _case(M=M, what="no csr")
        L = synth.make_layer(N=300, K=2048, bits=4, group_size=64, rank=16, density=0.005, seed=M)
        x = synth.make_activations(M, L.K, seed=M)
        y, H = run_prepared(vw, L, x, dora="fused", with_csr=False)
        check_close(y, oracle_product(L, x, H, with_csr=False), what=f"no csr M={M}")
        _case(M=M, what="heavy rows")
        Lh = synth.make_layer(N=256, K=3584, bits=4, group_size=128, rank=8, density=0.02, seed=11 + M,
                              heavy_frac=0.2, heavy_mult=10)
        xh = synth.make_activations(M, Lh.K, seed=M)
        y, H = run_prepared(vw, Lh, xh, dora="fused")
        check_close(y, oracle_product(Lh, xh, H), what=f"heavy M={M}")


def test_prepared_rank_sweep(vw):
    for r in (0, 8, 16, 64):
        for M in (1, 4):
            _case(r=r, M=M)
            L = synth.make_layer(N=272, K=2176, bits=4, group_size=128, rank=r, density=0.01, seed=r + M)
            x = synth.make_activations(M, L.K, seed=r)
            y, H = run_prepared(vw, L, x, dora="fused")
            check_close(y, oracle_product(L, x, H), what=f"r={r} M={M}")


def test_prepared_matches_reference_layout_path(vw):
    """Same layer through the prepared kernel and the reference-layout kernel."""
    L = synth.make_layer(N=1000, K=3584, bits=4, group_size=128, rank=16, density=0.005, seed=5)
    for M in (1, 3, 8):
        x = synth.make_activations(M, L.K, seed=M)
        a, H = run_prepared(vw, L, x, dora="fused")
        b, _ = run_product(vw, L, x, fused_h=True)
        check_close(a, b.astype(np.float64), tol=1.2e-3, what=f"prepared vs row layout M={M}")
        check_close(a, oracle_product(L, x, H), what=f"M={M}")


def test_prepared_deterministic_and_counters_reset(vw):
    """Repeated calls give identical bits; calls in a row (different inputs, split-K and
    fused H) leave the workspace's counters at zero."""
    L = synth.make_layer(N=96, K=8192, bits=4, group_size=128, rank=16, density=0.005, seed=3)
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, 4, 128, t["chunk_offsets"], t["chunk_cols"],
                               t["chunk_vals"])
    for M in (1, 4, 2, 32, 12, 1):
        x = synth.make_activations(M, L.K, seed=M + 40)
        a, H = run_prepared(vw, L, x, prep=prep, t=t)
        b, _ = run_prepared(vw, L, x, prep=prep, t=t)
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"M={M} not deterministic"
        check_close(a, oracle_product(L, x, H), what=f"M={M}")


def test_prepared_c_abi(vw):
    """wlq_prepare + wlq_gemm_prepared through ctypes, on a zero-filled workspace, twice
    in a row, then the counter area is checked to be zero again."""
    from qwen_wlqfastshot_helen_beta_amd import load_abi

    lib = load_abi()
    L = synth.make_layer(N=300, K=4096, bits=4, group_size=128, rank=8, density=0.005, seed=21)
    t = L.to_torch(DEV)
    stream = torch.cuda.current_stream().cuda_stream
    nbytes = lib.wlq_prepared_bytes(L.N, L.K, 4, 128, L.nnz)
    assert nbytes > 0
    prep = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    st = lib.wlq_prepare(t["q_packed"].data_ptr(), t["lut_c"].data_ptr(), L.N, L.K, 4, 128,
                         t["chunk_offsets"].data_ptr(), t["chunk_cols"].data_ptr(), t["chunk_vals"].data_ptr(), L.nnz,
                         prep.data_ptr(), nbytes, stream)
    assert st == 0, lib.wlq_last_error()
    for M in (1, 6):
        x = torch.from_numpy(synth.make_activations(M, L.K, seed=M)).to(DEV)
        ref, H = run_prepared(vw, L, x.cpu().numpy(), dora="fused")
        ws_bytes = lib.wlq_gemm_workspace_bytes(M, L.N, L.K, 4, 8, torch.cuda.current_device())
        ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=DEV)
        out = torch.empty((M, L.N), dtype=torch.float16, device=DEV)
        for rep in range(2):
            out.fill_(0)
            st = lib.wlq_gemm_prepared(x.data_ptr(), t["q_packed"].data_ptr(), t["lut_c"].data_ptr(), prep.data_ptr(),
                                       nbytes, out.data_ptr(), M, L.N, L.K, 4, L.wpr, 128,
                                       t["chunk_offsets"].data_ptr(), t["chunk_cols"].data_ptr(),
                                       t["chunk_vals"].data_ptr(), L.nnz, None, t["lora_B"].data_ptr(),
                                       t["dora_gamma"].data_ptr(), t["lora_A"].data_ptr(), 1.0, 8, ws.data_ptr(),
                                       ws.numel(), stream)
            assert st == 0, lib.wlq_last_error()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.view(np.uint16)), f"M={M} call {rep}"
            assert int(ws[:16384].count_nonzero()) == 0, "counters not reset"
        check_close(out.cpu().numpy(), oracle_product(L, x.cpu().numpy(), H), what=f"abi M={M}")
    # a buffer smaller than the layout is refused
    st = lib.wlq_gemm_prepared(x.data_ptr(), t["q_packed"].data_ptr(), t["lut_c"].data_ptr(), prep.data_ptr(),
                               nbytes - 256, out.data_ptr(), 6, L.N, L.K, 4, L.wpr, 128, t["chunk_offsets"].data_ptr(),
                               t["chunk_cols"].data_ptr(), t["chunk_vals"].data_ptr(), L.nnz, None,
                               t["lora_B"].data_ptr(), t["dora_gamma"].data_ptr(), t["lora_A"].data_ptr(), 1.0, 8,
                               ws.data_ptr(), ws.numel(), stream)
    assert st == 4


def test_prepared_graph_replay(vw):
    """The prepared product (fused H, split-K) captured in a HIP graph: every replay
    matches the eager result, with eager work and syncs between replays."""
    L = synth.make_layer(N=640, K=6144, bits=4, group_size=128, rank=16, density=0.005, seed=4)
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, 4, 128, t["chunk_offsets"], t["chunk_cols"],
                               t["chunk_vals"])
    vw.init_workspaces(L.N, L.K, torch.device(DEV))
    for M in (1, 4):
        x = torch.from_numpy(synth.make_activations(M, L.K, seed=8)).to(DEV)
        out = torch.empty((M, L.N), dtype=torch.float16, device=DEV)

        def step():
            if M == 1:
                torch.ops.wlq_fastShot.gemv(t["q_packed"], t["lut_c"], x[0], out[0], L.N, L.K, 4, t["chunk_offsets"],
                                            t["chunk_cols"], t["chunk_vals"], t["lora_B"], None, t["dora_gamma"], 1.0,
                                            128, t["lora_A"], prep)
            else:
                torch.ops.wlq_fastShot.gemm(x, t["q_packed"], t["lut_c"], out, L.N, L.K, 4, L.wpr, t["chunk_offsets"],
                                            t["chunk_cols"], t["chunk_vals"], None, t["lora_B"], t["dora_gamma"], 1.0,
                                            128, t["lora_A"], prep)

        step()
        torch.cuda.synchronize()
        eager = out.clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        for _ in range(4):
            out.zero_()
            step()  # eager work between replays
            torch.cuda.synchronize()
            out.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
