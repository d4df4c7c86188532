"""A synthetic Qwen2.5 checkpoint in the reference's on-disk WLQ format, loaded through the
vLLM plugin path (the single-GPU part of serving a WLQ model).

Writer: per decoder layer ``l`` one ``model-{l:05d}.safetensors`` with, for every projection
``p`` of ``self_attn`` (q, k, v, o) and ``mlp`` (gate, up, down), the tensors the plugin's
``create_weights`` registers (vllm_wlq/linear_method.py:376-411)::

    model.layers.{l}.{self_attn|mlp}.{p}_proj.q_packed        int32, continuous packing
    ...lut_c                                                   fp16 [N, 2**bits], one LUT per row
    ...bits                                                    int32 [1]
    ...ef_tile_size / ef_tile_meta / ef_bitstream              the outlier positions, Elias-Fano
    ...outlier_values                                          float8_e5m2, row-major position order

plus ``lora_adapter_distilled/adapter_model.safetensors`` (PEFT keys ``...{p}_proj.lora_A.weight``
[r, K] and ``lora_B.weight`` [N, r], fp16) and ``adapter_config.json`` (r, lora_alpha), which
``get_dora_adapter`` finds under the model directory (vllm_wlq/linear_method.py:17-120).
Codes are uniform, LUTs sorted metalog fits (synth.metalog_luts), outliers a uniform random
``density`` of the positions with N(0, 0.2) values; nothing is trained.

Loader: the vLLM model loader's part for the linears, without vLLM: per layer the merged
projections ``qkv_proj`` (shards q, k, v), ``o_proj``, ``gate_up_proj`` (shards 0, 1) and
``down_proj`` get ``create_weights``; every checkpoint tensor goes to its parameter's
``weight_loader`` with the shard id of the stacked-parameter mapping; then
``process_weights_after_loading`` (vllm_wlq/linear_method.py:123-183, :413-674).
"""
from __future__ import annotations

import json
import os
import time
from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

from . import formats, synth


@dataclass(frozen=True)
class ModelDims:
    hidden: int = 3584
    intermediate: int = 18944
    kv: int = 512          # k_proj / v_proj outputs (4 KV heads x 128)
    layers: int = 28


QWEN25_7B = ModelDims()

# projection -> (module, out features, in features) as functions of the dims
def _projections(d: ModelDims):
    return {
        "q_proj": ("self_attn", d.hidden, d.hidden),
        "k_proj": ("self_attn", d.kv, d.hidden),
        "v_proj": ("self_attn", d.kv, d.hidden),
        "o_proj": ("self_attn", d.hidden, d.hidden),
        "gate_proj": ("mlp", d.intermediate, d.hidden),
        "up_proj": ("mlp", d.intermediate, d.hidden),
        "down_proj": ("mlp", d.hidden, d.intermediate),
    }


# vLLM's merged linears and the stacked-parameter mapping (checkpoint projection -> (merged
# linear, shard id)) of its Qwen2 model
MERGED = {
    "qkv_proj": ("self_attn", ["q_proj", "k_proj", "v_proj"]),
    "o_proj": ("self_attn", ["o_proj"]),
    "gate_up_proj": ("mlp", ["gate_proj", "up_proj"]),
    "down_proj": ("mlp", ["down_proj"]),
}
STACKED = {"q_proj": ("qkv_proj", "q"), "k_proj": ("qkv_proj", "k"), "v_proj": ("qkv_proj", "v"),
           "o_proj": ("o_proj", None), "gate_proj": ("gate_up_proj", 0), "up_proj": ("gate_up_proj", 1),
           "down_proj": ("down_proj", None)}


def _random_codes_continuous(rng: np.random.Generator, N: int, K: int, bits: int) -> np.ndarray:
    """Continuous packing of N*K uniform codes, generated as words: uniform codes packed
    LSB first are uniform words (3-bit: 10 codes in the low 30 bits), and the tail of the
    last word is zero as the packer leaves it."""
    spw = formats.symbols_per_word(bits)
    total = N * K
    nwords = -(-total // spw)
    hi = (1 << (spw * bits)) - 1
    words = rng.integers(0, hi, size=nwords, dtype=np.uint32, endpoint=True)
    tail = total - (nwords - 1) * spw
    if tail < spw:
        words[-1] &= np.uint32((1 << (tail * bits)) - 1)
    return words


def _outliers(rng: np.random.Generator, N: int, K: int, density: float):
    """About density*N*K distinct positions (row-major order) and their e5m2 bytes."""
    want = int(round(density * N * K))
    if want == 0:
        z = np.zeros(0, dtype=np.int64)
        return z, z, np.zeros(0, dtype=np.uint8)
    flat = np.unique(rng.integers(0, N * K, size=want, dtype=np.int64))
    vals = formats.fp16_to_e5m2_u8((rng.standard_normal(flat.size) * 0.2).astype(np.float16))
    return flat // K, flat % K, vals


def write_synthetic_checkpoint(path: str, dims: ModelDims = QWEN25_7B, bits: int = 4, density: float = 0.005,
                               rank: int = 16, lora_alpha: float = 16.0, tile_size: int = 64,
                               seed: int = 0) -> Dict[str, object]:
    """Write the checkpoint and its adapter under ``path``; returns a summary (files, bytes)."""
    import torch
    from safetensors.torch import save_file

    os.makedirs(path, exist_ok=True)
    adir = os.path.join(path, "lora_adapter_distilled")
    os.makedirs(adir, exist_ok=True)
    rng = np.random.default_rng(seed)
    projs = _projections(dims)
    adapter = {}
    nbytes = 0
    for l in range(dims.layers):
        tensors = {}
        for p, (mod, N, K) in projs.items():
            pre = f"model.layers.{l}.{mod}.{p}"
            q = _random_codes_continuous(rng, N, K, bits)
            lut = synth.metalog_luts(rng, N, bits)
            rows, cols, vals = _outliers(rng, N, K, density)
            meta, stream = formats.ef_encode_coords(rows, cols, N, K, tile_size)
            tensors[f"{pre}.q_packed"] = torch.from_numpy(q.view(np.int32))
            tensors[f"{pre}.lut_c"] = torch.from_numpy(lut)
            tensors[f"{pre}.bits"] = torch.tensor([bits], dtype=torch.int32)
            tensors[f"{pre}.ef_tile_size"] = torch.tensor([tile_size], dtype=torch.int32)
            tensors[f"{pre}.ef_tile_meta"] = torch.from_numpy(meta)
            tensors[f"{pre}.ef_bitstream"] = torch.from_numpy(stream.view(np.int32))
            tensors[f"{pre}.outlier_values"] = torch.from_numpy(vals).view(torch.float8_e5m2)
            apre = f"base_model.model.model.layers.{l}.{mod}.{p}"
            adapter[f"{apre}.lora_A.weight"] = torch.from_numpy(
                (rng.standard_normal((rank, K), dtype=np.float32) * 0.01).astype(np.float16))
            adapter[f"{apre}.lora_B.weight"] = torch.from_numpy(
                (rng.standard_normal((N, rank), dtype=np.float32) * 0.01).astype(np.float16))
        fn = os.path.join(path, f"model-{l:05d}.safetensors")
        save_file(tensors, fn)
        nbytes += os.path.getsize(fn)
    save_file(adapter, os.path.join(adir, "adapter_model.safetensors"))
    with open(os.path.join(adir, "adapter_config.json"), "w") as f:
        json.dump({"r": rank, "lora_alpha": lora_alpha, "peft_type": "LORA", "use_dora": True}, f)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump({"model_type": "qwen2", "hidden_size": dims.hidden, "intermediate_size": dims.intermediate,
                   "num_hidden_layers": dims.layers, "kv_proj_size": dims.kv,
                   "quantization_config": {"quant_method": "wlq_fastshot", "bits": bits}}, f)
    return {"layers": dims.layers, "bytes": nbytes, "path": path}


@dataclass
class LoadedModel:
    layers: List[Dict[str, object]]   # per decoder layer: merged-linear name -> loaded module
    method: object                    # the WLQLinearMethod that loaded them
    seconds: Dict[str, float]         # read / weight_loader / process_weights_after_loading


def load_synthetic_checkpoint(path: str, dims: Optional[ModelDims] = None) -> LoadedModel:
    """Load ``path`` (written by write_synthetic_checkpoint) through create_weights ->
    weight_loader -> process_weights_after_loading, layer by layer."""
    import torch
    from safetensors import safe_open

    from .vllm_wlq.linear_method import WLQLinearMethod, reset_dora_cache
    from .vllm_wlq.quant_config import WLQFastShotConfig

    with open(os.path.join(path, "config.json")) as f:
        cfg = json.load(f)
    if dims is None:
        dims = ModelDims(hidden=cfg["hidden_size"], intermediate=cfg["intermediate_size"], kv=cfg["kv_proj_size"],
                         layers=cfg["num_hidden_layers"])
    bits = int(cfg.get("quantization_config", {}).get("bits", 4))
    reset_dora_cache()
    method = WLQLinearMethod(WLQFastShotConfig(bits=bits, model_id=path))
    projs = _projections(dims)
    t_read = t_load = t_proc = 0.0
    layers = []
    for l in range(dims.layers):
        mods = {}
        for name, (mod, parts) in MERGED.items():
            m = torch.nn.Module()
            outs = [projs[p][1] for p in parts]
            K = projs[parts[0]][2]
            method.create_weights(m, K, outs, K, sum(outs), torch.float16)
            m.vllm_prefix = f"model.layers.{l}.{mod}.{name}"
            mods[name] = m
        with safe_open(os.path.join(path, f"model-{l:05d}.safetensors"), framework="pt", device="cpu") as f:
            for key in f.keys():
                t1 = time.perf_counter()
                tensor = f.get_tensor(key)
                t2 = time.perf_counter()
                proj, pname = key.split(".")[-2:]
                target, shard = STACKED[proj]
                param = getattr(mods[target], pname)
                if shard is None:
                    param.weight_loader(param, tensor)
                else:
                    param.weight_loader(param, tensor, shard)
                t_read += t2 - t1
                t_load += time.perf_counter() - t2
        t3 = time.perf_counter()
        for m in mods.values():
            method.process_weights_after_loading(m)
        torch.cuda.synchronize()
        t_proc += time.perf_counter() - t3
        layers.append(mods)
    return LoadedModel(layers=layers, method=method,
                       seconds={"read": t_read, "weight_loader": t_load, "process_weights_after_loading": t_proc})


def linear_stack(model: LoadedModel, x_hidden, x_inter) -> None:
    """The model's quantized linears for one forward pass of M tokens: per layer qkv_proj,
    o_proj and gate_up_proj on x_hidden [M, hidden] and down_proj on x_inter [M, intermediate]
    (fixed inputs: the attention and activation between them are not part of this path)."""
    apply = model.method.apply
    for mods in model.layers:
        apply(mods["qkv_proj"], x_hidden)
        apply(mods["o_proj"], x_hidden)
        apply(mods["gate_up_proj"], x_hidden)
        apply(mods["down_proj"], x_inter)


def stack_bytes(dims: ModelDims = QWEN25_7B, bits: int = 4) -> int:
    """Code bytes of the quantized linears of all layers (the weight stream of one pass)."""
    tot = 0
    for _, N, K in _projections(dims).values():
        tot += N * formats.words_per_row(K, bits) * 4
    return tot * dims.layers
