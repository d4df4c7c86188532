"""GPU parity of the HIP kernels against the CPU oracle (small and ragged shapes).

Dequantization must be bit-exact; layer outputs must match within the stated
tolerance (see tests/gpu_helpers.py).
"""
import ctypes
import sys

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, check_close, oracle_product, oracle_w0, run_product
from oracle import wlq_oracle as O
from qwen_wlqfastshot_helen_beta_amd import synth

pytestmark = pytest.mark.gpu

GROUPS = {4: [0, 32, 64, 96, 128, 256], 3: [0, 64, 128], 2: [0, 64, 128], 1: [0, 128]}


def _case(bits, gs):
    print(f"[case] bits={bits} group_size={gs}", flush=True)


@pytest.mark.parametrize("bits", [4, 3, 2, 1])
def test_dequant_bit_exact(vw, bits):
    for gs in GROUPS[bits]:
        for density in (0.0, 0.02):
            _case(bits, gs)
            L = synth.make_layer(N=77, K=1000, bits=bits, group_size=gs, rank=0, density=density, seed=bits * 10 + gs)
            t = L.to_torch(DEV)
            W = torch.empty((L.N, L.K), dtype=torch.float16, device=DEV)
            vw._C.dequant_w0(t["q_packed"], t["lut_c"], W, L.N, L.K, bits, L.wpr, t["chunk_offsets"],
                             t["chunk_cols"], t["chunk_vals"], gs)
            torch.cuda.synchronize()
            got = W.cpu().numpy().view(np.uint16)
            ref = oracle_w0(L).view(np.uint16)
            assert np.array_equal(got, ref), f"bits={bits} gs={gs} d={density}: {int((got != ref).sum())} mismatches"


@pytest.mark.parametrize("M", [1, 2, 5, 16, 17, 32])
@pytest.mark.parametrize("bits", [4, 3])
def test_skinny_parity(vw, M, bits):
    for gs in GROUPS[bits]:
        _case(bits, gs)
        L = synth.make_layer(N=200, K=1408, bits=bits, group_size=gs, rank=8, density=0.01, seed=100 + M + gs)
        x = synth.make_activations(M, L.K, seed=M)
        y, H = run_product(vw, L, x)
        check_close(y, oracle_product(L, x, H), what=f"M={M} bits={bits} gs={gs}")
        # the reference's rounding points (fp16 GEMM output before the DoRA pass for M >= 16)
        check_close(y, oracle_product(L, x, H, round_gemm_output=None), what="reference rounding")


@pytest.mark.parametrize("bits", [2, 1])
def test_skinny_narrow_widths(vw, bits):
    for gs in GROUPS[bits]:
        for M in (1, 7):
            _case(bits, gs)
            L = synth.make_layer(N=130, K=1536, bits=bits, group_size=gs, rank=4, density=0.005, seed=7 + M)
            x = synth.make_activations(M, L.K, seed=3)
            y, H = run_product(vw, L, x)
            check_close(y, oracle_product(L, x, H), what=f"M={M} bits={bits} gs={gs}")


@pytest.mark.parametrize("M", [1, 9, 40])
def test_ragged_k_and_options(vw, M):
    """K not a multiple of 8 / of the slab, no outliers, no DoRA."""
    L = synth.make_layer(N=70, K=1001, bits=4, group_size=0, rank=4, density=0.01, seed=5)
    x = synth.make_activations(M, L.K, seed=9)
    for dora in (True, False):
        for csr in (True, False):
            y, H = run_product(vw, L, x, with_dora=dora, with_csr=csr)
            check_close(y, oracle_product(L, x, H, with_csr=csr), what=f"dora={dora} csr={csr}")


@pytest.mark.parametrize("M", [33, 64, 130, 257])
@pytest.mark.parametrize("bits", [4, 3])
def test_gemm_parity(vw, M, bits):
    for gs in GROUPS[bits]:
        _case(bits, gs)
        L = synth.make_layer(N=272, K=1280, bits=bits, group_size=gs, rank=16, density=0.01, seed=M + gs)
        x = synth.make_activations(M, L.K, seed=M)
        y, H = run_product(vw, L, x)
        check_close(y, oracle_product(L, x, H), what=f"M={M} bits={bits} gs={gs}")
        check_close(y, oracle_product(L, x, H, round_gemm_output=None), what="reference rounding")


def test_gemm_heavy_outlier_rows(vw):
    """Heavy-tailed CSR rows (more entries than the LDS staging holds for one chunk)."""
    L = synth.make_layer(N=256, K=1024, bits=4, group_size=64, rank=8, density=0.06, seed=11, heavy_frac=0.2,
                         heavy_mult=10)
    for M in (1, 8, 96):
        x = synth.make_activations(M, L.K, seed=M)
        y, H = run_product(vw, L, x)
        check_close(y, oracle_product(L, x, H), what=f"heavy M={M}")


def test_deterministic(vw):
    L = synth.make_layer(N=512, K=2048, bits=4, group_size=128, rank=16, density=0.005, seed=1)
    for M in (1, 16, 200):
        x = synth.make_activations(M, L.K, seed=2)
        a, _ = run_product(vw, L, x)
        b, _ = run_product(vw, L, x)
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"M={M} not deterministic"


def test_c_abi_matches_op(vw):
    """Call libwlq_hip.so directly through ctypes; same bits as the torch op."""
    from qwen_wlqfastshot_helen_beta_amd import load_abi

    lib = load_abi()
    L = synth.make_layer(N=300, K=2048, bits=4, group_size=128, rank=8, density=0.005, seed=21)
    t = L.to_torch(DEV)
    for M in (1, 12, 70):
        x = torch.from_numpy(synth.make_activations(M, L.K, seed=M)).to(DEV)
        H = torch.nn.functional.linear(x, t["lora_A"]).float()
        ref, _ = run_product(vw, L, x.cpu().numpy())
        out = torch.empty((M, L.N), dtype=torch.float16, device=DEV)
        nbytes = lib.wlq_gemm_workspace_bytes(M, L.N, L.K, 4, 0, torch.cuda.current_device())
        ws = torch.zeros(max(nbytes, 4), dtype=torch.uint8, device=DEV)  # zero-filled once, as documented
        stream = torch.cuda.current_stream().cuda_stream
        for rep in range(2):  # the second call relies on the first leaving the arrival counters at zero
            out.fill_(0)
            if M == 1:
                st = lib.wlq_gemv(t["q_packed"].data_ptr(), t["lut_c"].data_ptr(), x.data_ptr(), out.data_ptr(),
                                  t["chunk_offsets"].data_ptr(), t["chunk_cols"].data_ptr(),
                                  t["chunk_vals"].data_ptr(), t["lora_B"].data_ptr(), H.data_ptr(),
                                  t["dora_gamma"].data_ptr(), None, 1.0, 8, L.N, L.K, 4, 128, ws.data_ptr(),
                                  ws.numel(), stream)
            else:
                st = lib.wlq_gemm(x.data_ptr(), t["q_packed"].data_ptr(), t["lut_c"].data_ptr(), out.data_ptr(), M,
                                  L.N, L.K, 4, L.wpr, 128, t["chunk_offsets"].data_ptr(), t["chunk_cols"].data_ptr(),
                                  t["chunk_vals"].data_ptr(), H.data_ptr(), t["lora_B"].data_ptr(),
                                  t["dora_gamma"].data_ptr(), None, 1.0, 8, ws.data_ptr(), ws.numel(), stream)
            assert st == 0, lib.wlq_last_error()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.view(np.uint16)), f"M={M} call {rep}"
            if nbytes:
                assert int(ws[:16384].count_nonzero()) == 0, "arrival counters not reset"
        # fused H (lora_A) through the C ABI, twice on the same workspace
        if M <= 32:
            nb = lib.wlq_gemm_workspace_bytes(M, L.N, L.K, 4, 8, torch.cuda.current_device())
            wsf = torch.zeros(nb, dtype=torch.uint8, device=DEV)
            yf, Hf = run_product(vw, L, x.cpu().numpy(), fused_h=True)
            for rep in range(2):
                out.fill_(0)
                st = lib.wlq_gemm(x.data_ptr(), t["q_packed"].data_ptr(), t["lut_c"].data_ptr(), out.data_ptr(), M,
                                  L.N, L.K, 4, L.wpr, 128, t["chunk_offsets"].data_ptr(), t["chunk_cols"].data_ptr(),
                                  t["chunk_vals"].data_ptr(), None, t["lora_B"].data_ptr(),
                                  t["dora_gamma"].data_ptr(), t["lora_A"].data_ptr(), 1.0, 8, wsf.data_ptr(),
                                  wsf.numel(), stream)
                assert st == 0, lib.wlq_last_error()
                torch.cuda.synchronize()
                assert np.array_equal(out.cpu().numpy().view(np.uint16), yf.view(np.uint16)), f"fused M={M} {rep}"
                assert int(wsf[:16384].count_nonzero()) == 0, "arrival counters not reset (fused)"
        # no workspace at all is valid (no split-K)
        out2 = torch.empty_like(out)
        st = lib.wlq_gemm(x.data_ptr(), t["q_packed"].data_ptr(), t["lut_c"].data_ptr(), out2.data_ptr(), M, L.N,
                          L.K, 4, L.wpr, 128, t["chunk_offsets"].data_ptr(), t["chunk_cols"].data_ptr(),
                          t["chunk_vals"].data_ptr(), H.data_ptr(), t["lora_B"].data_ptr(), t["dora_gamma"].data_ptr(),
                          None, 1.0, 8, None, 0, stream)
        assert st == 0, lib.wlq_last_error()
        torch.cuda.synchronize()
        check_close(out2.cpu().numpy(), ref, what="no-workspace")


@pytest.mark.parametrize("M", [1, 5, 16, 32, 40, 130])
def test_fused_dora_h(vw, M):
    """lora_A passed instead of H: the product computes H = fp16(x A^T) itself
    (inside the decode kernel for M <= 32, with the lora_h kernel above)."""
    for bits, gs, r in ((4, 128, 16), (4, 0, 64), (3, 64, 8), (4, 64, 96)):
        L = synth.make_layer(N=260, K=2176, bits=bits, group_size=gs, rank=r, density=0.005, seed=M + r)
        x = synth.make_activations(M, L.K, seed=M)
        y, H = run_product(vw, L, x, fused_h=True)
        check_close(y, oracle_product(L, x, H), what=f"fused M={M} bits={bits} gs={gs} r={r}")


def test_fused_needs_workspace(vw):
    """Computing H from lora_A without a workspace is refused with WLQ_ERR_CAPACITY."""
    from qwen_wlqfastshot_helen_beta_amd import load_abi

    lib = load_abi()
    L = synth.make_layer(N=64, K=512, bits=4, group_size=128, rank=8, density=0.0, seed=1)
    t = L.to_torch(DEV)
    x = torch.from_numpy(synth.make_activations(1, L.K)).to(DEV)
    out = torch.empty((1, L.N), dtype=torch.float16, device=DEV)
    st = lib.wlq_gemv(t["q_packed"].data_ptr(), t["lut_c"].data_ptr(), x.data_ptr(), out.data_ptr(), None, None, None,
                      t["lora_B"].data_ptr(), None, t["dora_gamma"].data_ptr(), t["lora_A"].data_ptr(), 1.0, 8, L.N,
                      L.K, 4, 128, None, 0, torch.cuda.current_stream().cuda_stream)
    assert st == 4, st
    assert b"workspace" in lib.wlq_last_error()


def test_dora_epilogue_entry(vw):
    """wlq_dora_epilogue: in-place (fp16 out + s*H.B^T) * gamma (the reference's separate pass)."""
    from qwen_wlqfastshot_helen_beta_amd import load_abi

    lib = load_abi()
    rng = np.random.default_rng(3)
    M, N, r = 37, 300, 16
    y0 = rng.standard_normal((M, N)).astype(np.float16)
    H = rng.standard_normal((M, r)).astype(np.float16).astype(np.float32)
    B = (rng.standard_normal((N, r)) * 0.1).astype(np.float16)
    g = rng.uniform(0.9, 1.1, N).astype(np.float16)
    out = torch.from_numpy(y0.copy()).to(DEV)
    Ht, Bt, gt = (torch.from_numpy(a).to(DEV) for a in (H, B, g))
    st = lib.wlq_dora_epilogue(out.data_ptr(), Ht.data_ptr(), Bt.data_ptr(), gt.data_ptr(), 0.5, r, M, N,
                               torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    ref = ((y0.astype(np.float64) + 0.5 * (H.astype(np.float64) @ B.astype(np.float64).T))
           * g.astype(np.float64)).astype(np.float16)
    check_close(out.cpu().numpy(), ref, what="dora epilogue")


def test_graph_replay(vw):
    """The decode product captured in a HIP graph replays correctly (workspace pre-sized)."""
    L = synth.make_layer(N=1024, K=2048, bits=4, group_size=128, rank=16, density=0.005, seed=4)
    t = L.to_torch(DEV)
    vw.init_workspaces(L.N, L.K, torch.device(DEV))
    x = torch.from_numpy(synth.make_activations(1, L.K, seed=8)).to(DEV)
    out = torch.empty((1, L.N), dtype=torch.float16, device=DEV)

    def step():
        h = torch.nn.functional.linear(x[0], t["lora_A"]).float()
        torch.ops.wlq_fastShot.gemv(t["q_packed"], t["lut_c"], x[0], out[0], L.N, L.K, 4, t["chunk_offsets"],
                                    t["chunk_cols"], t["chunk_vals"], t["lora_B"], h, t["dora_gamma"], 1.0, 128)

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
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
