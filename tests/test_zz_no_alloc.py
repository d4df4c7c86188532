"""wlq_gemm_prepared_noalloc (no workspace argument: the library's per-GPU scratch)
against wlq_gemm_prepared (a caller's zero-filled workspace of the same size, so both
plan the same kernels): bit-identical outputs on consecutive calls, the second with a
smaller input; M = 64 through the M = 9..128 kernel; a call whose plan needs more than the
scratch is refused before anything is launched."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import DEV
from qwen_wlqfastshot_helen_beta_amd import synth

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20  # the library's scratch per GPU
vp = ctypes.c_void_p


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _layer(vw, N, K, seed):
    L = synth.make_layer(N=N, K=K, bits=4, group_size=128, rank=16, density=0.005, seed=seed)
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, 4, 128, t["chunk_offsets"], t["chunk_cols"],
                               t["chunk_vals"])
    assert prep.numel() > 0
    return L, t, prep


def _args(L, t, prep, x, out):
    """Arguments shared by both entry points, up to (not including) the workspace."""
    return [vp(x.data_ptr()), vp(t["q_packed"].data_ptr()), vp(t["lut_c"].data_ptr()), vp(prep.data_ptr()),
            prep.numel(), vp(out.data_ptr()), x.shape[0], L.N, L.K, 4, L.wpr, 128, vp(t["chunk_offsets"].data_ptr()),
            vp(t["chunk_cols"].data_ptr()), vp(t["chunk_vals"].data_ptr()), L.nnz, None, vp(t["lora_B"].data_ptr()),
            vp(t["dora_gamma"].data_ptr()), vp(t["lora_A"].data_ptr()), 1.0, L.rank]


def _both(lib, L, t, prep, M, seed, ws):
    x = torch.from_numpy(synth.make_activations(M, L.K, seed=seed)).to(DEV)
    stream = vp(torch.cuda.current_stream().cuda_stream)
    out_ws = torch.full((M, L.N), 7.0, dtype=torch.float16, device=DEV)
    out_na = torch.full((M, L.N), 7.0, dtype=torch.float16, device=DEV)
    st = lib.wlq_gemm_prepared(*_args(L, t, prep, x, out_ws), vp(ws.data_ptr()), ws.numel(), stream)
    assert st == 0, lib.wlq_last_error()
    st = lib.wlq_gemm_prepared_noalloc(*_args(L, t, prep, x, out_na), stream)
    assert st == 0, lib.wlq_last_error()
    torch.cuda.synchronize()
    a, b = out_ws.cpu().numpy(), out_na.cpu().numpy()
    assert np.isfinite(a.astype(np.float32)).all()
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"M={M} N={L.N}: outputs differ"


def test_noalloc_matches_workspace_entry(vw):
    from qwen_wlqfastshot_helen_beta_amd import load_abi

    lib = load_abi()
    ws = torch.zeros(SCRATCH_BYTES, dtype=torch.uint8, device=DEV)  # same size: same plans
    gate = _layer(vw, 18944, 3584, seed=11)
    small = _layer(vw, 512, 3584, seed=12)
    _case("noalloc: gate 18944x3584 M=4, then k 512x3584 M=1 (smaller)")
    _both(lib, *gate, 4, 1, ws)
    _both(lib, *small, 1, 2, ws)
    _case("noalloc: again, gate M=8 then k M=2")
    _both(lib, *gate, 8, 3, ws)
    _both(lib, *small, 2, 4, ws)
    _case("noalloc: M=64 (H from lora_A in the scratch), then M=1")
    _both(lib, *small, 64, 5, ws)
    _both(lib, *small, 1, 6, ws)


def test_noalloc_refuses_beyond_scratch(vw):
    """A 16640 x 16512 layer at M = 128 runs the M = 9..128 kernel with two K splits (129
    slabs, more than one split holds): 17 MB of split partials, beyond the scratch.  The
    layer's contents do not matter for a refusal, so it is made on the device (no outliers)."""
    from qwen_wlqfastshot_helen_beta_amd import load_abi

    lib = load_abi()
    N, K, M, r = 16640, 16512, 128, 16
    _case("noalloc: 16640x16512 M=128 needs > 16 MiB of split partials: refused, nothing launched")
    g = torch.Generator(device=DEV)
    g.manual_seed(13)
    wpr = K // 8
    q = torch.randint(-2**31, 2**31 - 1, (N, wpr), dtype=torch.int32, device=DEV, generator=g)
    lut = torch.randn(N, K // 128, 16, generator=g, device=DEV).half()
    A = torch.randn(r, K, generator=g, device=DEV).half()
    B = torch.randn(N, r, generator=g, device=DEV).half()
    gamma = torch.ones(N, device=DEV).half()
    prep = vw._C.prepare_layer(q, lut, N, K, 4, 128)
    assert prep.numel() > 0
    x = torch.randn(M, K, generator=g, device=DEV).half()
    out = torch.full((M, N), 7.0, dtype=torch.float16, device=DEV)
    torch.cuda.synchronize()
    st = lib.wlq_gemm_prepared_noalloc(vp(x.data_ptr()), vp(q.data_ptr()), vp(lut.data_ptr()), vp(prep.data_ptr()),
                                       prep.numel(), vp(out.data_ptr()), M, N, K, 4, wpr, 128, None, None, None, 0,
                                       None, vp(B.data_ptr()), vp(gamma.data_ptr()), vp(A.data_ptr()), 1.0, r,
                                       vp(torch.cuda.current_stream().cuda_stream))
    assert st == 4, (st, lib.wlq_last_error())  # WLQ_ERR_CAPACITY
    assert b"scratch" in lib.wlq_last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()), "a refused call must not write the output"
    del q, lut, A, B, gamma, prep, x, out
    torch.cuda.empty_cache()
    L, t, prep = _layer(vw, 18944, 3584, seed=13)
    # the scratch is untouched by the refusal: a following call still matches
    ws = torch.zeros(SCRATCH_BYTES, dtype=torch.uint8, device=DEV)
    _both(lib, L, t, prep, 2, 8, ws)
