"""vLLM symbols used by the plugin, with stand-ins when vLLM is not installed.

With vLLM present these are vLLM's own classes, so the plugin registers and
behaves exactly like the reference (vllm_wlq/quant_config.py:1-12,
vllm_wlq/linear_method.py:11-15).  Without it, minimal stand-ins keep the
module importable so the layer can be driven directly (tests, benchmarks).
"""
from __future__ import annotations

import torch

try:  # pragma: no cover - vLLM is not part of this image
    from vllm.model_executor.layers.quantization import register_quantization_config
    from vllm.model_executor.layers.quantization.base_config import QuantizationConfig
    from vllm.model_executor.layers.linear import (
        LinearBase,
        LinearMethodBase,
        RowParallelLinear,
        ColumnParallelLinear,
        UnquantizedLinearMethod,
    )

    HAVE_VLLM = True
except Exception:  # ImportError or a broken install
    HAVE_VLLM = False

    def register_quantization_config(name: str):
        def deco(cls):
            return cls

        return deco

    class QuantizationConfig:  # noqa: D401 - stand-in
        """Stand-in for vllm...base_config.QuantizationConfig."""

    class LinearBase(torch.nn.Module):
        """Stand-in for vllm's LinearBase."""

    class RowParallelLinear(LinearBase):
        pass

    class ColumnParallelLinear(LinearBase):
        pass

    class LinearMethodBase:
        pass

    class UnquantizedLinearMethod(LinearMethodBase):
        pass


def get_tp_info():
    """(tp_rank, tp_size); (0, 1) outside a vLLM tensor-parallel group
    (vllm_wlq/linear_method.py:341-346)."""
    try:
        from vllm.distributed import get_tensor_model_parallel_rank, get_tensor_model_parallel_world_size

        return get_tensor_model_parallel_rank(), get_tensor_model_parallel_world_size()
    except Exception:
        return 0, 1
