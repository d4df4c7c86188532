"""A synthetic checkpoint in the reference's on-disk format, written by checkpoint.py, loaded
through create_weights -> weight_loader -> process_weights_after_loading
(vllm_wlq/linear_method.py:123-183, :413-674) for vLLM's merged projections, and applied:
every merged linear of every layer against the CPU oracle built independently from the
files (continuous codes unpacked, Elias-Fano tiles decoded, adapter merged, gamma from
||W0|| as the reference computes it without a magnitude vector), and the whole linear stack
under one HIP graph replaying to the eager result."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, check_close
from oracle import wlq_oracle as O
from qwen_wlqfastshot_helen_beta_amd import checkpoint as C

pytestmark = pytest.mark.gpu

SMALL = C.ModelDims(hidden=384, intermediate=1024, kv=128, layers=2)
RANK, ALPHA = 8, 16.0


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _oracle_layer(path, l, name):
    """(W0 fp16 [N, K], A, B, m=None) of merged linear `name` of layer l, from the files."""
    from safetensors import safe_open

    mod, parts = C.MERGED[name]
    projs = C._projections(SMALL)
    W0s, As, Bs = [], [], []
    with safe_open(str(path / f"model-{l:05d}.safetensors"), framework="pt") as f, \
            safe_open(str(path / "lora_adapter_distilled" / "adapter_model.safetensors"), framework="pt") as fa:
        get = lambda key: f.get_tensor(key).numpy()  # noqa: E731
        for p in parts:
            _, N, K = projs[p]
            pre = f"model.layers.{l}.{mod}.{p}"
            codes = O.unpack_continuous(get(f"{pre}.q_packed").view(np.uint32), N, K, 4)
            q, _ = O.pack_row_aligned(codes, 4)
            T = int(get(f"{pre}.ef_tile_size")[0])
            off, cols = O.ef_decode_to_chunk_csr(get(f"{pre}.ef_tile_meta"), get(f"{pre}.ef_bitstream").view(np.uint32),
                                                 N, K, T, 512)
            vals = f.get_tensor(f"{pre}.outlier_values").view(torch.uint8).numpy()
            W0s.append(O.dequant(q, get(f"{pre}.lut_c"), N, K, 4, off, cols, vals))
            apre = f"base_model.model.model.layers.{l}.{mod}.{p}"
            As.append(fa.get_tensor(f"{apre}.lora_A.weight").numpy())
            Bs.append(fa.get_tensor(f"{apre}.lora_B.weight").numpy())
    A, B, _ = O.merge_dora(As, Bs, [None] * len(As))
    return np.concatenate(W0s), A, B


def test_checkpoint_load_and_apply(vw, tmp_path):
    _case("write 2-layer checkpoint")
    C.write_synthetic_checkpoint(str(tmp_path), SMALL, bits=4, density=0.01, rank=RANK, lora_alpha=ALPHA,
                                 tile_size=64, seed=5)
    _case("load through the plugin")
    model = C.load_synthetic_checkpoint(str(tmp_path))
    assert len(model.layers) == 2 and all(v >= 0 for v in model.seconds.values())
    s = O.lora_scale(ALPHA, RANK)
    rng = np.random.default_rng(0)
    for l in range(SMALL.layers):
        for name, mod in model.layers[l].items():
            W0, A, B = _oracle_layer(tmp_path, l, name)
            assert mod.has_dora and abs(mod.lora_scale - s) < 1e-12
            assert mod.lora_A_f16.shape[0] == RANK * len(C.MERGED[name][1])
            g_ref = O.dora_gamma(W0, A, B, s, None)
            g = mod.dora_gamma.cpu().numpy()
            dg = np.abs(g.view(np.uint16).astype(np.int32) - g_ref.view(np.uint16).astype(np.int32))
            assert dg.max() <= 1, f"layer {l} {name}: gamma off by {dg.max()} ulp"
            A16, B16 = A.astype(np.float16), B.astype(np.float16)
            for M in (1, 6, 24, 100):
                _case(f"layer {l} {name} M={M}")
                x = rng.standard_normal((M, W0.shape[1])).astype(np.float16)
                y = model.method.apply(mod, torch.from_numpy(x).to(DEV)).cpu().numpy()
                check_close(y, O.apply(x, W0, A16, B16, g, s), what=f"layer {l} {name} M={M}")

    _case("linear stack: eager vs graph replay")
    xh = torch.randn(8, SMALL.hidden, device=DEV).half()
    xi = torch.randn(8, SMALL.intermediate, device=DEV).half()
    outs = []
    orig_apply = model.method.apply

    def recording_apply(layer, x, bias=None):
        y = orig_apply(layer, x, bias)
        outs.append(y)
        return y

    model.method.apply = recording_apply
    C.linear_stack(model, xh, xi)
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    outs.clear()
    s_ = torch.cuda.Stream()
    s_.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s_):
        C.linear_stack(model, xh, xi)
    torch.cuda.current_stream().wait_stream(s_)
    torch.cuda.synchronize()
    outs.clear()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        C.linear_stack(model, xh, xi)
    graph_outs = list(outs)
    for rep in range(2):
        for o in graph_outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(graph_outs, eager):
            assert torch.equal(a, b), f"replay {rep}"
    model.method.apply = orig_apply
