"""GPU tests of the vLLM plugin path: load-time processing of a checkpoint-format
layer (continuous codes, EF-coded and 1-bit-mask outliers, a DoRA adapter
directory) and ``WLQLinearMethod.apply`` end to end (fp16/bf16, bias, 3-D input),
against the CPU oracle."""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, REL_TOL, check_close
from oracle import wlq_oracle as O
from qwen_wlqfastshot_helen_beta_amd import synth

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _write_adapter(tmp_path, layer_idx, parts, K, r, alpha, rng):
    """lora_adapter_distilled/ with PEFT-style keys for the given (name, N) projections."""
    from safetensors.torch import save_file

    d = tmp_path / "lora_adapter_distilled"
    d.mkdir()
    tensors, As, Bs, Ms = {}, [], [], []
    for name, N in parts:
        A = (rng.standard_normal((r, K)) * 0.05).astype(np.float16)
        B = (rng.standard_normal((N, r)) * 0.05).astype(np.float16)
        m = rng.uniform(0.5, 2.0, N).astype(np.float32)
        pre = f"base_model.model.model.layers.{layer_idx}.mlp.{name}"
        tensors[f"{pre}.lora_A.weight"] = torch.from_numpy(A)
        tensors[f"{pre}.lora_B.weight"] = torch.from_numpy(B)
        tensors[f"{pre}.lora_magnitude_vector"] = torch.from_numpy(m)
        As.append(A)
        Bs.append(B)
        Ms.append(m)
    save_file(tensors, str(d / "adapter_model.safetensors"))
    (d / "adapter_config.json").write_text(json.dumps({"r": r, "lora_alpha": alpha}))
    return As, Bs, Ms


@pytest.mark.parametrize("fmt", ["ef", "mask1bit"])
def test_process_weights_after_loading_and_apply(vw, tmp_path, fmt):
    from qwen_wlqfastshot_helen_beta_amd.vllm_wlq.linear_method import WLQLinearMethod, reset_dora_cache

    rng = np.random.default_rng(7)
    K, r, alpha, tile = 704, 8, 16, 32
    parts = [("gate_proj", 96), ("up_proj", 64)]
    As, Bs, Ms = _write_adapter(tmp_path, 3, parts, K, r, alpha, rng)
    reset_dora_cache()
    method = WLQLinearMethod(vw.WLQFastShotConfig(bits=4, model_id=str(tmp_path)))
    layer = torch.nn.Module()
    method.create_weights(layer, K, [n for _, n in parts], K, sum(n for _, n in parts), torch.float16)
    layer.vllm_prefix = "model.layers.3.mlp.gate_up_proj"

    W0_parts = []
    for s, (name, N) in enumerate(parts):
        _case(f"load shard {s} {name} ({fmt})")
        codes = rng.integers(0, 16, (N, K)).astype(np.uint8)
        lut = np.sort(rng.standard_normal((N, 16)) * 0.02, axis=1).astype(np.float16)
        mask = rng.random((N, K)) < 0.01
        vals16 = (rng.standard_normal(int(mask.sum())) * 0.2).astype(np.float16)
        e5 = O.fp16_bits_to_e5m2(vals16.view(np.uint16))
        load = lambda pname, t: getattr(layer, pname).weight_loader(getattr(layer, pname), t, s)
        load("q_packed", torch.from_numpy(O.pack_continuous(codes, 4).view(np.int32)))
        load("lut_c", torch.from_numpy(lut))
        load("bits", torch.tensor([4], dtype=torch.int32))
        if fmt == "ef":  # Elias-Fano tiles
            meta, stream = O.ef_encode(mask, tile)
            load("ef_tile_meta", torch.from_numpy(np.asarray(meta, np.int64)))
            load("ef_bitstream", torch.from_numpy(np.asarray(stream, np.uint32).view(np.int32)))
            load("ef_tile_size", torch.tensor([tile], dtype=torch.int32))
        else:  # 1-bit packed mask
            load("outlier_mask_1bit", torch.from_numpy(np.packbits(mask.ravel())))
        load("outlier_values", torch.from_numpy(e5).view(torch.float8_e5m2))
        q, _ = O.pack_row_aligned(codes, 4)
        off, cols, v = O.build_chunk_csr(mask, e5, 512)
        W0_parts.append(O.dequant(q, lut, N, K, 4, off, cols, v))
    method.process_weights_after_loading(layer)
    W0 = np.concatenate(W0_parts)
    N = W0.shape[0]

    # load-time products: row-aligned codes, CSR and the dequant are bit-exact
    W_dev = torch.empty((N, K), dtype=torch.float16, device=DEV)
    vw._C.dequant_w0(layer.q_packed_aligned, layer.lut_c, W_dev, N, K, 4, layer.words_per_row, layer.chunk_offsets,
                     layer.chunk_cols, layer.chunk_vals)
    torch.cuda.synchronize()
    assert np.array_equal(W_dev.cpu().numpy().view(np.uint16), W0.view(np.uint16))

    # DoRA merge and gamma (fp32 on the GPU vs fp64 oracle: within one fp16 ulp)
    A, B, m = O.merge_dora(As, Bs, Ms)
    s = O.lora_scale(alpha, r)
    assert layer.has_dora and abs(layer.lora_scale - s) < 1e-12
    assert np.array_equal(layer.lora_A_f16.cpu().numpy().astype(np.float64), A)
    assert np.array_equal(layer.lora_B.cpu().numpy().astype(np.float64), B)
    g_ref = O.dora_gamma(W0, A, B, s, m)
    g = layer.dora_gamma.cpu().numpy()
    assert np.max(np.abs(g.view(np.uint16).astype(np.int32) - g_ref.view(np.uint16).astype(np.int32))) <= 1

    # apply end to end
    A16, B16 = A.astype(np.float16), B.astype(np.float16)
    for M in (1, 5, 40):
        _case(f"apply fp16 M={M}")
        x = (rng.standard_normal((M, K))).astype(np.float16)
        y = method.apply(layer, torch.from_numpy(x).to(DEV)).cpu().numpy()
        ref = O.apply(x, W0, A16, B16, g, s)
        check_close(y, ref, what=f"apply M={M}")
    _case("apply bf16 3-D with bias")
    xb = torch.randn(2, 3, K, device=DEV, dtype=torch.bfloat16)
    bias = torch.randn(N, device=DEV, dtype=torch.bfloat16)
    yb = method.apply(layer, xb, bias)
    assert yb.dtype == torch.bfloat16 and yb.shape == (2, 3, N)
    ref = O.apply(xb.float().cpu().numpy(), W0, A16, B16, g, s, bias=bias.float().cpu().numpy(),
                  out_dtype=np.float32)
    # bf16 output: compare with bf16's own resolution (2^-8 relative) on top of the layer tolerance
    y64 = yb.float().cpu().numpy().astype(np.float64)
    r64 = ref.astype(np.float64)
    assert O.rel_err(y64, r64) <= REL_TOL + 2.0 ** -8


def test_apply_without_dora_and_config0(vw):
    """Config 0 shape (Qwen2.5-0.5B up_proj 4864x896), per-row LUT, no adapter; M=1 and M=64."""
    from qwen_wlqfastshot_helen_beta_amd.vllm_wlq.linear_method import WLQLinearMethod, attach_synthetic

    N, K = synth.QWEN25_05B_UP_PROJ
    for gs in (0, 128):
        L = synth.make_layer(N, K, bits=4, group_size=gs, rank=8, density=0.005, seed=0)
        W0 = O.dequant(L.q, L.lut, L.N, L.K, 4, L.offsets, L.cols, L.vals, group_size=gs)
        method = WLQLinearMethod(vw.WLQFastShotConfig(bits=4, group_size=gs))
        layer = attach_synthetic(torch.nn.Module(), L, torch.device(DEV))
        for M in (1, 64):
            _case(f"config0 gs={gs} M={M}")
            x = synth.make_activations(M, K, seed=M)
            y = method.apply(layer, torch.from_numpy(x).to(DEV)).cpu().numpy()
            check_close(y, O.apply(x, W0, L.A, L.B, L.gamma, L.lora_scale), what=f"cfg0 gs={gs} M={M}")
            layer.has_dora = False
            y = method.apply(layer, torch.from_numpy(x).to(DEV)).cpu().numpy()
            check_close(y, O.apply(x, W0), what=f"cfg0 no-dora gs={gs} M={M}")
            layer.has_dora = True
