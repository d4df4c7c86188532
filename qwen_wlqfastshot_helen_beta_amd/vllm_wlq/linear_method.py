"""``WLQLinearMethod``: the quantized linear layer behind vLLM's LinearBase.

Same methods and layer attributes as the reference (vllm_wlq/linear_method.py:372-1009):

* ``create_weights`` registers the checkpoint parameters (packed codes, LUTs,
  bit width, Elias-Fano or 1-bit outlier masks, outlier values) with a
  shard-stashing weight loader;
* ``process_weights_after_loading`` converts them to the device format
  (row-aligned codes, padded LUTs, chunk-CSR outliers, merged DoRA factors and
  the calibrated magnitude scale gamma) -- host conversions run in the native
  ``_C`` helpers, gamma uses the device dequantization ``_C.dequant_w0``;
* ``apply`` runs one forward: fp16 activations, then
  ``torch.ops.wlq_fastShot.gemv`` (one row) or ``.gemm`` (several rows) with
  ``lora_A`` so the DoRA ``H = fp16(x A^T)`` is computed inside the product
  (the reference computes it with a separate F.linear), cast back to the
  caller's dtype and bias added in that dtype.

Tensor parallelism (the reference's general path, :676-935) is handled by vLLM
sharding outside this module on multi-GPU deployments and is not part of this
single-GPU build: ``process_weights_after_loading`` raises for tp_size > 1.
"""
from __future__ import annotations

import json
import math
import os
import re
from typing import Any, Dict, List, Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

from .. import formats
from . import _C
from ._vllm_compat import LinearMethodBase, RowParallelLinear, get_tp_info

# Module-level helpers under the reference's names.
pack_indices_row_aligned = formats.pack_indices_row_aligned
build_chunk_csr_np = formats.build_chunk_csr

_DORA_CACHE: Optional[Tuple[Dict[Tuple[int, str], list], Dict[str, Any]]] = None

PROJ_NAMES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj", "in_proj_qkvz",
              "in_proj_qkv", "in_proj_z", "in_proj_ba", "in_proj_b", "in_proj_a", "out_proj")


def unpack_indices_continuous(q_packed_tensor: torch.Tensor, N: int, M: int, bits: int) -> np.ndarray:
    """Continuous on-disk packing -> codes [N, M] (vllm_wlq/linear_method.py:315-323)."""
    return formats.unpack_indices_continuous(q_packed_tensor.cpu().numpy(), N, M, bits)


def build_chunk_csr(mask_2d: np.ndarray, fp8_values_raw: torch.Tensor, chunk_m: int):
    """Dense mask -> (chunk_offsets, chunk_cols, chunk_vals) tensors (vllm_wlq/linear_method.py:284-312)."""
    vals = fp8_values_raw.cpu()
    if vals.numel() == 0:
        v_np = np.zeros(0, dtype=np.uint8)
    elif vals.dtype == torch.float16:
        v_np = vals.numpy()
    else:
        v_np = vals.contiguous().view(torch.uint8).numpy()
    off, cols, v = formats.build_chunk_csr(mask_2d, v_np, chunk_m)
    if vals.numel() == 0:
        v = np.zeros(0, dtype=np.uint8)
    return torch.from_numpy(off), torch.from_numpy(cols.view(np.int16)).view(torch.uint16), torch.from_numpy(v)


def decode_elias_fano(ef_tile_meta: np.ndarray, ef_bitstream_u32: np.ndarray, orig_shape, tile_size: int = 32):
    """Per-tile Elias-Fano bitstreams -> dense bool mask (vllm_wlq/linear_method.py:243-281)."""
    H, W = orig_shape
    Hp, Wp = -(-H // tile_size) * tile_size, -(-W // tile_size) * tile_size
    nty, ntx = Hp // tile_size, Wp // tile_size
    U = tile_size * tile_size
    tiles = np.zeros((nty * ntx, U), dtype=bool)
    bits = np.unpackbits(np.ascontiguousarray(ef_bitstream_u32).view(np.uint8), bitorder="little")
    meta = np.asarray(ef_tile_meta, dtype=np.int64).reshape(-1, 2)
    for k in range(min(meta.shape[0], nty * ntx)):
        start, m = int(meta[k, 0]), int(meta[k, 1])
        if m <= 0:
            continue
        L = max(0, int(math.floor(math.log2(U / m)))) if U > m else 0
        if L > 0:
            low = (bits[start:start + m * L].reshape(m, L).astype(np.int64) << np.arange(L, dtype=np.int64)).sum(1)
        else:
            low = np.zeros(m, dtype=np.int64)
        ones = np.flatnonzero(bits[start + m * L:start + m * L + m + ((U - 1) >> L) + 1])[:m]
        high = ones - np.arange(ones.size, dtype=np.int64)
        idx = (high << L) | low[:ones.size]
        tiles[k, idx[idx < U]] = True
    mask = tiles.reshape(nty, ntx, tile_size, tile_size).swapaxes(1, 2).reshape(Hp, Wp)
    return mask[:H, :W]


def get_dora_adapter(model_id_or_path: Optional[str] = None):
    """Find ``lora_adapter_distilled/adapter_model.safetensors`` (+ adapter_config.json)
    locally and index its tensors by (layer, projection) -> [lora_A, lora_B, magnitude].

    Candidate directories follow vllm_wlq/linear_method.py:29-51.  Remote
    downloads (:53-79) are not attempted (offline deployments).  Cached per process.
    """
    global _DORA_CACHE
    if _DORA_CACHE is not None:
        return _DORA_CACHE
    cands = ["lora_adapter_distilled", "./lora_adapter_distilled", "../lora_adapter_distilled",
             "mtg_0.01_pct_relMSE_shot/lora_adapter_distilled", "mtg_0.01_pct_relMSE_shot_ef/lora_adapter_distilled"]
    if model_id_or_path and os.path.isdir(model_id_or_path):
        cands = [os.path.join(model_id_or_path, "lora_adapter_distilled"), model_id_or_path] + cands
    weights: Dict[str, torch.Tensor] = {}
    config: Dict[str, Any] = {}
    for d in cands:
        af = os.path.join(d, "adapter_model.safetensors")
        if os.path.isfile(af):
            from safetensors import safe_open

            with safe_open(af, framework="pt", device="cpu") as f:
                for k in f.keys():
                    weights[k] = f.get_tensor(k)
            cf = os.path.join(d, "adapter_config.json")
            if os.path.isfile(cf):
                with open(cf, "r", encoding="utf-8") as fh:
                    config = json.load(fh)
            break
    index: Dict[Tuple[int, str], list] = {}
    layer_re = re.compile(r"layers\.(\d+)\.")
    for k, v in weights.items():
        lm = layer_re.search(k)
        if not lm:
            continue
        li = int(lm.group(1))
        kl = k.lower()
        for p in PROJ_NAMES:
            if f".{p}." in k or k.endswith(f".{p}"):
                slot = index.setdefault((li, p), [None, None, None])
                if "lora_a" in kl:
                    slot[0] = v
                elif "lora_b" in kl:
                    slot[1] = v
                elif "dora_scale" in kl or "magnitude_vector" in kl:
                    slot[2] = v
    _DORA_CACHE = (index, config)
    return _DORA_CACHE


def reset_dora_cache() -> None:
    global _DORA_CACHE
    _DORA_CACHE = None


def flexible_weight_loader(param: torch.nn.Parameter, loaded_weight: torch.Tensor, *args, **kwargs):
    """Stash every loaded shard on the parameter (vllm_wlq/linear_method.py:123-137)."""
    shard_id = args[0] if len(args) > 0 else kwargs.get("shard_id", None)
    if not hasattr(param, "_shard_dict"):
        param._shard_dict = {}
    if not hasattr(param, "_shard_list"):
        param._shard_list = []
    if hasattr(torch, "float8_e5m2") and loaded_weight.dtype == torch.float8_e5m2:
        loaded_weight = loaded_weight.view(torch.uint8)
    if shard_id is not None:
        param._shard_dict[shard_id] = loaded_weight
    param._shard_list.append(loaded_weight)
    param.data = loaded_weight
    param._is_loaded = True


def create_layer_weight_param(layer: torch.nn.Module, data: torch.Tensor):
    param = torch.nn.Parameter(data, requires_grad=False)
    param.weight_loader = flexible_weight_loader
    param._shard_dict = {}
    param._shard_list = []
    param._is_loaded = False
    return param


def _shard_sort_key(k):
    if isinstance(k, int):
        return (0, k)
    if isinstance(k, (tuple, list)) and len(k) > 0:
        return (0, int(k[0]))
    order = {"q": 0, "k": 1, "v": 2, "gate": 0, "up": 1}
    return (1, order.get(str(k), 99))


def get_shards_in_order(param, layer=None) -> List[torch.Tensor]:
    """Loaded shards in q,k,v / gate,up order (vllm_wlq/linear_method.py:163-183)."""
    if param is None or not getattr(param, "_is_loaded", False):
        return []
    d = getattr(param, "_shard_dict", {})
    if d:
        return [d[k] for k in sorted(d.keys(), key=_shard_sort_key)]
    lst = getattr(param, "_shard_list", [])
    if lst:
        return lst
    return [param.data] if param.data.numel() > 0 else []


def _sub_projections(prefix: str, dora_index) -> List[str]:
    lm = re.search(r"layers\.(\d+)\.", prefix)
    if not lm:
        return []
    li = int(lm.group(1))
    if "in_proj_qkvz" in prefix:
        return ["in_proj_qkvz"] if (li, "in_proj_qkvz") in dora_index else ["in_proj_qkv", "in_proj_z"]
    if "in_proj_ba" in prefix:
        return ["in_proj_ba"] if (li, "in_proj_ba") in dora_index else ["in_proj_b", "in_proj_a"]
    for key, subs in (("in_proj_qkv", ["in_proj_qkv"]), ("qkv_proj", ["q_proj", "k_proj", "v_proj"]),
                      ("gate_up_proj", ["gate_proj", "up_proj"]), ("out_proj", ["out_proj"]),
                      ("o_proj", ["o_proj"]), ("down_proj", ["down_proj"])):
        if key in prefix:
            return subs
    return []


def _to_e5m2_u8(v: torch.Tensor) -> torch.Tensor:
    v = v.cpu()
    if v.dtype == torch.float16:
        return torch.from_numpy(formats.fp16_to_e5m2_u8(v.numpy()))
    return v.contiguous().view(torch.uint8)


def calibrate_dora_gamma(W0: torch.Tensor, A: torch.Tensor, B: torch.Tensor, scale: float,
                         magnitude: Optional[torch.Tensor]) -> torch.Tensor:
    """gamma = fp16(m / max(||W0 + s B A||_row, 1e-12)), m defaulting to ||W0||_row,
    computed in fp32 on W0's device (vllm_wlq/linear_method.py:625-635)."""
    with torch.no_grad():
        W = W0.float()
        V = W + scale * (B.to(W.device, torch.float32) @ A.to(W.device, torch.float32))
        norm_v = torch.norm(V, p=2, dim=1).clamp(min=1e-12)
        if magnitude is not None and magnitude.numel() == W.shape[0]:
            m = magnitude.flatten().to(W.device, torch.float32)
        else:
            m = torch.norm(W, p=2, dim=1)
        return (m / norm_v).to(torch.float16)


class WLQLinearMethod(LinearMethodBase):
    _MAX_N: int = 0
    _MAX_K: int = 0

    def __init__(self, quant_config):
        self.quant_config = quant_config

    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int, output_partition_sizes: List[int],
                       input_size: int, output_size: int, params_dtype: torch.dtype, **extra_kwargs):
        layer.output_partition_sizes = list(output_partition_sizes)
        layer.N = int(sum(output_partition_sizes))
        layer.K = int(input_size_per_partition)
        fp8_t = getattr(torch, "float8_e5m2", torch.uint8)
        for name, dt in (("weight", torch.float16), ("q_packed", torch.int32), ("lut_c", torch.float16),
                         ("bits", torch.int32), ("orig_shape", torch.int32), ("is_quantized", torch.uint8),
                         ("ef_tile_size", torch.int32), ("ef_tile_meta", torch.int64), ("ef_bitstream", torch.int32),
                         ("outlier_mask_1bit", torch.uint8), ("outlier_mask", torch.uint8),
                         ("outlier_values", fp8_t), ("fp8_outliers", fp8_t), ("outliers", fp8_t)):
            layer.register_parameter(name, create_layer_weight_param(layer, torch.empty(0, dtype=dt)))

    # ------------------------------------------------------------------ load
    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        device = torch.device(f"cuda:{torch.cuda.current_device()}") if torch.cuda.is_available() else None
        if device is None:
            raise RuntimeError("WLQLinearMethod needs a ROCm GPU; no CPU fallback exists")
        tp_rank, tp_size = get_tp_info()
        if tp_size != 1:
            raise NotImplementedError("tensor-parallel loading is outside this single-GPU build")
        cfg = self.quant_config
        group_size = int(getattr(cfg, "group_size", 0) or 0)

        def shards(name):
            return get_shards_in_order(getattr(layer, name, None), layer)

        q_sh, lut_sh, bits_sh = shards("q_packed"), shards("lut_c"), shards("bits")
        meta_sh, stream_sh, tile_sh = shards("ef_tile_meta"), shards("ef_bitstream"), shards("ef_tile_size")
        mask_sh, vals_sh = shards("outlier_mask_1bit"), shards("outlier_values")
        out_sizes = getattr(layer, "output_partition_sizes", [layer.N])
        if lut_sh and all(t.dim() >= 2 and t.shape[0] > 0 for t in lut_sh):
            part = [int(t.shape[0]) for t in lut_sh]
        elif len(q_sh) == 1 and len(out_sizes) > 1:
            part = [int(sum(out_sizes))]
        else:
            part = [int(s) for s in out_sizes]
        K = int(layer.K)

        bits_list = []
        for s in range(len(part)):
            if bits_sh:
                b_t = bits_sh[s] if s < len(bits_sh) else bits_sh[0]
                bits_list.append(int(b_t.item()) if b_t.numel() > 0 else cfg.bits)
            else:
                bits_list.append(cfg.bits)
        bits = max(bits_list) if bits_list else cfg.bits
        ncb = 1 << bits
        chunk_m = formats.chunk_width(bits)
        nch = formats.num_chunks(K, bits)

        q_parts, lut_parts, off_parts, col_parts, val_parts = [], [], [], [], []
        running = 0
        wpr = formats.words_per_row(K, bits)
        for s, N_s in enumerate(part):
            b_s = bits_list[s]
            q_raw = (q_sh[s] if s < len(q_sh) else layer.q_packed.data).cpu()
            if b_s == bits:
                q_al, wpr = _C.repack_q_indices_row_aligned(q_raw, N_s, K, bits)
            else:  # widen a narrower shard to the layer width
                codes = formats.unpack_indices_continuous(q_raw.numpy(), N_s, K, b_s)
                packed, wpr = formats.pack_indices_row_aligned(codes, bits)
                q_al = torch.from_numpy(packed.view(np.int32))
            q_parts.append(q_al)
            lut_s = (lut_sh[s] if s < len(lut_sh) else layer.lut_c.data).cpu().to(torch.float16)
            if lut_s.shape[-1] < ncb:
                lut_s = F.pad(lut_s, (0, ncb - lut_s.shape[-1]), value=0.0)
            lut_parts.append(lut_s.reshape(N_s, -1))
            tile_sz = 64
            if tile_sh:
                t_t = tile_sh[s] if s < len(tile_sh) else tile_sh[0]
                if t_t.numel() > 0:
                    tile_sz = int(t_t.item())
            if s < len(meta_sh) and meta_sh[s].numel() > 0 and s < len(stream_sh) and stream_sh[s].numel() > 0:
                off_s, col_s = _C.decode_ef_to_chunk_csr(meta_sh[s], stream_sh[s], N_s, K, tile_sz, chunk_m)
            elif s < len(mask_sh) and mask_sh[s].numel() > 0:
                m_s = np.unpackbits(mask_sh[s].cpu().numpy())[:N_s * K].reshape(N_s, K).astype(bool)
                off_s, col_s, _ = build_chunk_csr(m_s, torch.empty(0, dtype=torch.uint8), chunk_m)
            else:
                off_s = torch.zeros((N_s, nch + 1), dtype=torch.int32)
                col_s = torch.empty(0, dtype=torch.uint16)
            if running:
                off_s = off_s + running
            running += int(col_s.numel())
            off_parts.append(off_s)
            col_parts.append(col_s)
            if s < len(vals_sh) and vals_sh[s].numel() > 0:
                val_parts.append(_to_e5m2_u8(vals_sh[s]))
            else:
                val_parts.append(torch.zeros(int(col_s.numel()), dtype=torch.uint8))

        q_all = torch.cat(q_parts) if len(q_parts) > 1 else q_parts[0]
        lut_all = torch.cat(lut_parts) if len(lut_parts) > 1 else lut_parts[0]
        offsets = torch.cat(off_parts) if len(off_parts) > 1 else off_parts[0]
        cols = torch.cat([c.view(torch.int16) for c in col_parts]).view(torch.uint16)
        vals = torch.cat(val_parts) if len(val_parts) > 1 else val_parts[0]
        if vals.numel() != cols.numel():
            raise ValueError(f"outlier values ({vals.numel()}) do not match decoded positions ({cols.numel()})")

        q_dev = q_all.to(device)
        lut_dev = lut_all.to(device).contiguous()
        off_dev = offsets.to(device).contiguous()
        col_dev = cols.to(device)
        val_dev = vals.to(device)

        has_dora, A16, B16, gamma, scale = self._load_dora(layer, q_dev, lut_dev, off_dev, col_dev, val_dev, bits,
                                                            wpr, group_size, device)

        for name in ("weight", "q_packed", "lut_c", "outlier_mask_1bit", "outlier_mask", "outlier_values",
                     "fp8_outliers", "outliers", "ef_tile_meta", "ef_bitstream", "ef_tile_size", "orig_shape",
                     "is_quantized", "dora_scale", "bits"):
            if name in getattr(layer, "_parameters", {}):
                del layer._parameters[name]
            if hasattr(layer, name):
                try:
                    delattr(layer, name)
                except Exception:
                    pass

        layer.q_packed_aligned = q_dev
        layer.words_per_row = int(wpr)
        layer.lut_c = lut_dev
        layer.quant_bits = bits
        layer.wlq_group_size = group_size
        layer.chunk_offsets = off_dev
        layer.chunk_cols = col_dev
        layer.chunk_vals = val_dev
        layer.has_dora = has_dora
        layer.lora_A_f16 = A16 if has_dora else None
        layer.lora_B = B16
        layer.dora_gamma = gamma
        layer.lora_scale = scale
        layer.wlq_prepared = prepare_layer(layer)
        if layer.N > WLQLinearMethod._MAX_N or layer.K > WLQLinearMethod._MAX_K:
            WLQLinearMethod._MAX_N = max(WLQLinearMethod._MAX_N, layer.N)
            WLQLinearMethod._MAX_K = max(WLQLinearMethod._MAX_K, layer.K)
            _C.init_workspaces(WLQLinearMethod._MAX_N, WLQLinearMethod._MAX_K, device)

    def _load_dora(self, layer, q_dev, lut_dev, off_dev, col_dev, val_dev, bits, wpr, group_size, device):
        """Merge the adapter factors and calibrate gamma (vllm_wlq/linear_method.py:533-639)."""
        index, acfg = get_dora_adapter(getattr(self.quant_config, "model_id", None))
        none = (False, None, None, None, 1.0)
        if not index:
            return none
        subs = _sub_projections(getattr(layer, "vllm_prefix", ""), index)
        lm = re.search(r"layers\.(\d+)\.", getattr(layer, "vllm_prefix", ""))
        if not subs or lm is None:
            return none
        li = int(lm.group(1))
        As, Bs, Ms = [], [], []
        for p in subs:
            e = index.get((li, p))
            if e and e[0] is not None and e[1] is not None:
                As.append(e[0].float())
                Bs.append(e[1].float())
                Ms.append(e[2].float() if e[2] is not None else None)
        if len(As) != len(subs):
            return none
        r_base = Bs[0].shape[1]
        scale = float(acfg.get("lora_alpha", r_base)) / float(r_base)
        if len(subs) == 1:
            A, B, m = As[0], Bs[0], Ms[0]
        else:
            A = torch.cat(As, dim=0)
            B = torch.block_diag(*Bs)
            m = torch.cat([x.flatten() for x in Ms]) if all(x is not None for x in Ms) else None
        if B.shape[0] != layer.N or A.shape[1] != layer.K:
            return none  # shape mismatch disables DoRA (vllm_wlq/linear_method.py:594-596)
        W0 = torch.empty((layer.N, layer.K), dtype=torch.float16, device=device)
        _C.dequant_w0(q_dev, lut_dev, W0, layer.N, layer.K, bits, wpr, off_dev, col_dev, val_dev, group_size)
        gamma = calibrate_dora_gamma(W0, A, B, scale, m)
        del W0
        A16 = A.to(device=device, dtype=torch.float16).contiguous()
        B16 = B.to(device=device, dtype=torch.float16).contiguous()
        return True, A16, B16, gamma.contiguous(), scale

    # ----------------------------------------------------------------- forward
    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        orig_shape = x.shape
        orig_dtype = x.dtype
        x2 = x.reshape(-1, layer.K)
        if x2.dtype != torch.float16:
            x2 = x2.to(torch.float16)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        M = x2.shape[0]
        out = torch.empty((M, layer.N), dtype=torch.float16, device=x.device)
        has_dora = bool(getattr(layer, "has_dora", False)) and getattr(layer, "lora_A_f16", None) is not None
        lora_B = layer.lora_B if has_dora else None
        gamma = layer.dora_gamma if has_dora else None
        bits = int(getattr(layer, "quant_bits", self.quant_config.bits))
        gs = int(getattr(layer, "wlq_group_size", 0))
        scale = float(getattr(layer, "lora_scale", 1.0))
        A = layer.lora_A_f16 if has_dora else None
        prep = getattr(layer, "wlq_prepared", None)
        if M == 1:
            # H = fp32(fp16(x A^T)) is computed inside the product from lora_A
            torch.ops.wlq_fastShot.gemv(layer.q_packed_aligned, layer.lut_c, x2.squeeze(0), out.squeeze(0), layer.N,
                                        layer.K, bits, layer.chunk_offsets, layer.chunk_cols, layer.chunk_vals,
                                        lora_B, None, gamma, scale, gs, A, prep)
        else:
            torch.ops.wlq_fastShot.gemm(x2, layer.q_packed_aligned, layer.lut_c, out, layer.N, layer.K, bits,
                                        layer.words_per_row, layer.chunk_offsets, layer.chunk_cols, layer.chunk_vals,
                                        None, lora_B, gamma, scale, gs, A, prep)
        y = out if orig_dtype == torch.float16 else out.to(orig_dtype)
        if bias is not None:
            y.add_(bias)
        return y.view(*orig_shape[:-1], layer.N)


def attach_synthetic(layer: torch.nn.Module, synth, device, prepared: bool = True) -> torch.nn.Module:
    """Put a ``synth.SynthLayer`` onto ``layer`` in the post-load device format
    (what process_weights_after_loading produces), for benchmarks and tests."""
    t = synth.to_torch(device)
    layer.N, layer.K = synth.N, synth.K
    layer.q_packed_aligned = t["q_packed"]
    layer.words_per_row = synth.wpr
    layer.lut_c = t["lut_c"]
    layer.quant_bits = synth.bits
    layer.wlq_group_size = synth.group_size
    layer.chunk_offsets = t["chunk_offsets"]
    layer.chunk_cols = t["chunk_cols"]
    layer.chunk_vals = t["chunk_vals"]
    layer.has_dora = synth.B is not None
    layer.lora_A_f16 = t.get("lora_A")
    layer.lora_B = t.get("lora_B")
    layer.dora_gamma = t.get("dora_gamma")
    layer.lora_scale = synth.lora_scale
    layer.wlq_prepared = prepare_layer(layer) if prepared else None
    return layer


def prepare_layer(layer: torch.nn.Module) -> Optional[torch.Tensor]:
    """The layer's load-time tile-contiguous layout for the decode kernel (None when
    its format has none: only 4- and 3-bit codes with a per-row LUT or a group size
    that is a multiple of 32, K % 8 == 0).  Built on the device from the reference-format tensors, which
    the layer keeps for the other kernels and for dequant_w0."""
    t = _C.prepare_layer(layer.q_packed_aligned, layer.lut_c, layer.N, layer.K, int(layer.quant_bits),
                         int(getattr(layer, "wlq_group_size", 0)), layer.chunk_offsets, layer.chunk_cols,
                         layer.chunk_vals)
    return t if t.numel() > 0 else None
