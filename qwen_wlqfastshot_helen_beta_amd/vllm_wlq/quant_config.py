"""``WLQFastShotConfig``: the vLLM quantization config of the plugin.

Same registry names, methods and prefix rules as the reference
(vllm_wlq/quant_config.py:10-82).  ``bits`` is the fallback width when a layer
carries no ``bits`` tensor; ``chunk_m`` is always 640 for 3-bit and 512
otherwise, as the kernels require.  ``group_size`` (0 = one LUT per output row)
is this build's extension and defaults to the reference layout.
"""
from __future__ import annotations

from typing import Any, Dict, List, Optional

import torch

from ._vllm_compat import LinearBase, QuantizationConfig, UnquantizedLinearMethod, register_quantization_config

DEFAULT_MODEL_ID = "wichtel-labs/Qwen3.8-27B-WLQ-FastShot"


@register_quantization_config("wlq_fastshot")
@register_quantization_config("wlq_fastShot")
class WLQFastShotConfig(QuantizationConfig):
    """Metalog FastShot (wlq_fastShot) quantization settings."""

    def __init__(self, bits: int = 4, outlier_fraction: float = 0.05, chunk_m: int = 512, use_dora: bool = True,
                 model_id: Optional[str] = None, group_size: int = 0):
        super().__init__()
        self.bits = bits
        self.outlier_fraction = outlier_fraction
        self.chunk_m = 640 if bits == 3 else chunk_m
        self.use_dora = use_dora
        self.model_id = model_id or DEFAULT_MODEL_ID
        self.group_size = int(group_size or 0)

    def __repr__(self) -> str:
        return (f"WLQFastShotConfig(bits={self.bits}, outlier_fraction={self.outlier_fraction}, "
                f"chunk_m={self.chunk_m}, use_dora={self.use_dora}, group_size={self.group_size})")

    def get_name(self) -> str:
        return "wlq_fastShot"

    def get_supported_act_dtypes(self) -> List[torch.dtype]:
        return [torch.float16, torch.bfloat16]

    @classmethod
    def get_min_capability(cls) -> int:
        return 80

    @classmethod
    def get_config_filenames(cls) -> List[str]:
        return ["/config.json"]

    @classmethod
    def from_config(cls, config: Dict[str, Any]) -> "WLQFastShotConfig":
        q_cfg = config.get("quantization_config") or config
        bits = q_cfg.get("bits", 4)
        return cls(
            bits=bits,
            outlier_fraction=q_cfg.get("outlier_fraction", 0.05),
            chunk_m=640 if bits == 3 else q_cfg.get("chunk_m", 512),
            use_dora=q_cfg.get("use_dora", True),
            model_id=config.get("_name_or_path", DEFAULT_MODEL_ID),
            group_size=q_cfg.get("group_size", 0),
        )

    def get_quant_method(self, layer: torch.nn.Module, prefix: str) -> Optional[Any]:
        if not isinstance(layer, LinearBase):
            return None
        if prefix.startswith("model.visual") or "visual" in prefix or "blocks." in prefix or "lm_head" in prefix:
            return UnquantizedLinearMethod()
        if any(s in prefix for s in ("conv1d", "router", "shared_expert_gate")):
            return UnquantizedLinearMethod()
        layer.vllm_prefix = prefix
        from .linear_method import WLQLinearMethod

        return WLQLinearMethod(self)

    def get_scaled_act_names(self) -> List[str]:
        return []
