"""Failure reporting of the decode kernels' cross-block hand-offs, with the failing
condition forced from the host so that every kernel still exits normally:

* the wait for the fused DoRA H runs out of polls: a subprocess sets the library's
  test hooks (WLQ_TEST_HOOKS=1 before its first product, then WLQ_TEST_WITHHOLD_H=1
  keeps the DoRA finisher from raising its ready slots, WLQ_SPIN_LIMIT=64 polls);
* counters not zero at entry (two unordered calls on one workspace, or a workspace
  never zero-filled): the host writes large counts into a caller-owned workspace
  and calls through the C ABI.

In both cases the rows concerned come back as NaN, wlq_workspace_status /
check_workspaces report WLQ_ERR_SYNC, later calls on the workspace keep writing
NaN (the error word is sticky) and wlq_workspace_reset restores normal results."""
from __future__ import annotations

import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from gpu_helpers import DEV
from qwen_wlqfastshot_helen_beta_amd import synth

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SYNC_BYTES = 16384
ERROR_WORD = SYNC_BYTES // 4 - 32  # the counter area's last 128-byte line

_TIMEOUT_SCRIPT = r"""
import os, sys
sys.path.insert(0, os.environ["WLQ_ROOT"])
import numpy as np, torch
import qwen_wlqfastshot_helen_beta_amd.vllm_wlq as vw
from qwen_wlqfastshot_helen_beta_amd import synth
dev = torch.device("cuda:0")
L = synth.make_layer(N=512, K=1024, bits=4, group_size=128, rank=16, density=0.005, seed=3)
t = L.to_torch(dev)
prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, 4, 128, t["chunk_offsets"], t["chunk_cols"],
                           t["chunk_vals"])
x = torch.from_numpy(synth.make_activations(1, L.K, seed=1)).to(dev)
def run():
    out = torch.empty(1, L.N, dtype=torch.float16, device=dev)
    torch.ops.wlq_fastShot.gemv(t["q_packed"], t["lut_c"], x[0], out[0], L.N, L.K, 4, t["chunk_offsets"],
                                t["chunk_cols"], t["chunk_vals"], t["lora_B"], None, t["dora_gamma"], 1.0, 128,
                                t["lora_A"], prep)
    torch.cuda.synchronize()
    return out.cpu().numpy()
print("[sub] normal call", flush=True)
y0 = run()
assert np.isfinite(y0.astype(np.float32)).all()
vw.check_workspaces(dev)
print("[sub] withheld ready slots", flush=True)
os.environ["WLQ_TEST_WITHHOLD_H"] = "1"
y1 = run()
assert np.isnan(y1.astype(np.float32)).all(), "timed-out waits must write NaN rows"
try:
    vw.check_workspaces(dev)
    raise AssertionError("check_workspaces did not report the timeout")
except RuntimeError as e:
    assert "ran out of polls" in str(e), str(e)
print("[sub] sticky error", flush=True)
os.environ["WLQ_TEST_WITHHOLD_H"] = "0"
y2 = run()
assert np.isnan(y2.astype(np.float32)).all(), "the error word must poison later calls"
print("[sub] reset", flush=True)
vw.reset_workspaces(dev)
y3 = run()
assert np.array_equal(y3.view(np.uint16), y0.view(np.uint16)), "results after reset differ"
vw.check_workspaces(dev)
print("[sub] ok", flush=True)
"""


def test_h_wait_timeout_is_reported_and_poisons(vw):
    env = dict(os.environ, WLQ_TEST_HOOKS="1", WLQ_SPIN_LIMIT="64", WLQ_TEST_WITHHOLD_H="0", WLQ_ROOT=ROOT)
    print("[case] H-wait timeout (subprocess, test hooks)", flush=True)
    p = subprocess.run([sys.executable, "-c", _TIMEOUT_SCRIPT], env=env, stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True, timeout=150)
    print(p.stdout, flush=True)
    assert p.returncode == 0, p.stdout[-2000:]
    assert "[sub] ok" in p.stdout


def _abi_call(lib, L, t, x, out, ws, prepared, H):
    vp = ctypes.c_void_p
    stream = torch.cuda.current_stream().cuda_stream
    if prepared is not None:
        st = lib.wlq_gemm_prepared(vp(x.data_ptr()), vp(t["q_packed"].data_ptr()), vp(t["lut_c"].data_ptr()),
                                   vp(prepared.data_ptr()), prepared.numel(), vp(out.data_ptr()), x.shape[0], L.N,
                                   L.K, L.bits, L.wpr, L.group_size, vp(t["chunk_offsets"].data_ptr()),
                                   vp(t["chunk_cols"].data_ptr()), vp(t["chunk_vals"].data_ptr()), L.nnz,
                                   vp(H.data_ptr()), vp(t["lora_B"].data_ptr()), vp(t["dora_gamma"].data_ptr()),
                                   None, 1.0, L.rank, vp(ws.data_ptr()), ws.numel(), vp(stream))
    else:
        st = lib.wlq_gemm(vp(x.data_ptr()), vp(t["q_packed"].data_ptr()), vp(t["lut_c"].data_ptr()),
                          vp(out.data_ptr()), x.shape[0], L.N, L.K, L.bits, L.wpr, L.group_size,
                          vp(t["chunk_offsets"].data_ptr()), vp(t["chunk_cols"].data_ptr()),
                          vp(t["chunk_vals"].data_ptr()), vp(H.data_ptr()), vp(t["lora_B"].data_ptr()),
                          vp(t["dora_gamma"].data_ptr()), None, 1.0, L.rank, vp(ws.data_ptr()), ws.numel(),
                          vp(stream))
    assert st == 0, lib.wlq_last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy().copy()


@pytest.mark.parametrize("layout", ["prepared", "row"])
def test_stale_counters_are_reported_and_poison(vw, layout):
    """A narrow layer (512 x 3584: several K splits at M = 1, so the tile blocks hand their
    partials over through the counters), H given by the caller."""
    from qwen_wlqfastshot_helen_beta_amd import load_abi

    lib = load_abi()
    print(f"[case] stale counters, {layout} layout", flush=True)
    L = synth.make_layer(N=512, K=3584, bits=4, group_size=128, rank=16, density=0.005, seed=4)
    t = L.to_torch(DEV)
    prep = None
    if layout == "prepared":
        prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, 4, 128, t["chunk_offsets"],
                                   t["chunk_cols"], t["chunk_vals"])
    x = torch.from_numpy(synth.make_activations(1, L.K, seed=2)).to(DEV)
    H = torch.nn.functional.linear(x, t["lora_A"]).float().contiguous()
    need = lib.wlq_gemm_workspace_bytes(1, L.N, L.K, 4, 0, 0)
    ws = torch.zeros(max(need, SYNC_BYTES) + 4096, dtype=torch.uint8, device=DEV)
    out = torch.empty(1, L.N, dtype=torch.float16, device=DEV)
    y0 = _abi_call(lib, L, t, x, out, ws, prep, H)
    assert np.isfinite(y0.astype(np.float32)).all()
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.wlq_workspace_status(ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(stream)) == 0
    # every counter far beyond what one call reaches (the error word itself stays 0)
    ws[:ERROR_WORD * 4].view(torch.int32).fill_(1 << 20)
    torch.cuda.synchronize()
    y1 = _abi_call(lib, L, t, x, out, ws, prep, H)
    assert np.isnan(y1.astype(np.float32)).any(), "overflowing arrivals must write NaN rows"
    st = lib.wlq_workspace_status(ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(stream))
    assert st == 7, (st, lib.wlq_last_error())
    assert b"exceeded" in lib.wlq_last_error()
    y2 = _abi_call(lib, L, t, x, out, ws, prep, H)
    assert np.isnan(y2.astype(np.float32)).all(), "the sticky error word must poison the next call"
    assert lib.wlq_workspace_reset(ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(stream)) == 0
    y3 = _abi_call(lib, L, t, x, out, ws, prep, H)
    assert np.array_equal(y3.view(np.uint16), y0.view(np.uint16)), "results after reset differ"
    assert lib.wlq_workspace_status(ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(stream)) == 0


def test_workspace_per_stream(vw):
    """Products on two streams use two workspaces (no shared counters); results match."""
    print("[case] two streams", flush=True)
    L = synth.make_layer(N=512, K=3584, bits=4, group_size=128, rank=16, density=0.005, seed=5)
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, 4, 128, t["chunk_offsets"], t["chunk_cols"],
                               t["chunk_vals"])
    x = torch.from_numpy(synth.make_activations(4, L.K, seed=3)).to(DEV)
    outs = []
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for s in streams:
        with torch.cuda.stream(s):
            o = torch.empty(4, L.N, dtype=torch.float16, device=DEV)
            for _ in range(20):
                torch.ops.wlq_fastShot.gemm(x, t["q_packed"], t["lut_c"], o, L.N, L.K, 4, L.wpr, t["chunk_offsets"],
                                            t["chunk_cols"], t["chunk_vals"], None, t["lora_B"], t["dora_gamma"],
                                            1.0, 128, t["lora_A"], prep)
            outs.append(o)
    torch.cuda.synchronize()
    vw.check_workspaces(torch.device(DEV))
    a, b = (o.cpu().numpy() for o in outs)
    assert np.isfinite(a.astype(np.float32)).all()
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_workspace_created_under_capture(vw):
    """A stream's first product inside graph capture: its workspace is created there (the
    counter fill is recorded, not run), zeroed again before the stream's next eager call,
    and every replay and eager call matches the eager result of another stream."""
    print("[case] workspace created under capture", flush=True)
    L = synth.make_layer(N=1024, K=3584, bits=4, group_size=128, rank=16, density=0.005, seed=6)
    t = L.to_torch(DEV)
    prep = vw._C.prepare_layer(t["q_packed"], t["lut_c"], L.N, L.K, 4, 128, t["chunk_offsets"], t["chunk_cols"],
                               t["chunk_vals"])
    x = torch.from_numpy(synth.make_activations(1, L.K, seed=4)).to(DEV)
    out = torch.empty(1, L.N, dtype=torch.float16, device=DEV)

    def step():
        torch.ops.wlq_fastShot.gemv(t["q_packed"], t["lut_c"], x[0], out[0], L.N, L.K, 4, t["chunk_offsets"],
                                    t["chunk_cols"], t["chunk_vals"], t["lora_B"], None, t["dora_gamma"], 1.0, 128,
                                    t["lora_A"], prep)

    step()
    torch.cuda.synchronize()
    eager = out.clone()
    cap = torch.cuda.Stream()  # never used eagerly before the capture
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        step()
    torch.cuda.synchronize()
    out.zero_()
    with torch.cuda.stream(cap):
        step()  # eager on the capture stream before any replay
    torch.cuda.synchronize()
    assert torch.equal(out, eager)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        out.zero_()
        with torch.cuda.stream(cap):
            step()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    vw.check_workspaces(torch.device(DEV))
