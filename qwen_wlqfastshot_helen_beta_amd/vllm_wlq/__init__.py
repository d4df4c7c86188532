"""vLLM plugin ``wlq_fastShot``: metalog-LUT weight quantization on MI355X.

Registers the custom ops ``torch.ops.wlq_fastShot.gemv`` and ``.gemm`` with the
reference's schemas (vllm_wlq/__init__.py:9-74) -- ``out`` is mutated in place,
fake implementations keep them traceable for graph capture and torch.compile --
plus trailing defaulted arguments: ``group_size`` (0 = one LUT per row),
``lora_A`` (when lora_h / lora_H is None, the op computes the DoRA H itself as
fp32(fp16(x @ lora_A^T)), the reference caller's F.linear) and ``prepared``
(the layer's load-time tile-contiguous layout from ``_C.prepare_layer``, which the
product kernels read for every M: codes, LUT planes and outlier patch lists).
Both call the ``_C`` extension, which calls the C ABI of ``libwlq_hip.so``.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _C  # noqa: F401  (no fallback: the product path needs the HIP extension)


def _register_ops() -> None:
    ns = "wlq_fastShot"
    if hasattr(torch.ops, ns) and hasattr(getattr(torch.ops, ns), "gemv") and hasattr(getattr(torch.ops, ns), "gemm"):
        return  # already registered by another import path of this package

    @torch.library.custom_op(f"{ns}::gemv", mutates_args={"out"})
    def _gemv_op(
        q_packed: torch.Tensor,
        lut_c: torch.Tensor,
        x: torch.Tensor,
        out: torch.Tensor,
        N: int,
        K: int,
        bits: int,
        chunk_offsets: Optional[torch.Tensor] = None,
        chunk_cols: Optional[torch.Tensor] = None,
        chunk_vals: Optional[torch.Tensor] = None,
        lora_B: Optional[torch.Tensor] = None,
        lora_h: Optional[torch.Tensor] = None,
        dora_gamma: Optional[torch.Tensor] = None,
        lora_scale: float = 1.0,
        group_size: int = 0,
        lora_A: Optional[torch.Tensor] = None,
        prepared: Optional[torch.Tensor] = None,
    ) -> None:
        _C.gemv_forward(q_packed, lut_c, x, out, int(N), int(K), int(bits), chunk_offsets, chunk_cols, chunk_vals,
                        lora_B, lora_h, dora_gamma, float(lora_scale), int(group_size), lora_A, prepared)

    @_gemv_op.register_fake
    def _gemv_fake(q_packed, lut_c, x, out, N, K, bits, chunk_offsets=None, chunk_cols=None, chunk_vals=None,
                   lora_B=None, lora_h=None, dora_gamma=None, lora_scale=1.0, group_size=0, lora_A=None,
                   prepared=None):
        return None

    @torch.library.custom_op(f"{ns}::gemm", mutates_args={"out"})
    def _gemm_op(
        X: torch.Tensor,
        q_packed: torch.Tensor,
        lut_c: torch.Tensor,
        out: torch.Tensor,
        N: int,
        K: int,
        bits: int,
        words_per_row: int,
        chunk_offsets: Optional[torch.Tensor] = None,
        chunk_cols: Optional[torch.Tensor] = None,
        chunk_vals: Optional[torch.Tensor] = None,
        lora_H: Optional[torch.Tensor] = None,
        lora_B: Optional[torch.Tensor] = None,
        dora_gamma: Optional[torch.Tensor] = None,
        lora_scale: float = 1.0,
        group_size: int = 0,
        lora_A: Optional[torch.Tensor] = None,
        prepared: Optional[torch.Tensor] = None,
    ) -> None:
        _C.gemm_forward(X, q_packed, lut_c, out, int(N), int(K), int(bits), int(words_per_row), chunk_offsets,
                        chunk_cols, chunk_vals, lora_H, lora_B, dora_gamma, float(lora_scale), int(group_size), lora_A,
                        prepared)

    @_gemm_op.register_fake
    def _gemm_fake(X, q_packed, lut_c, out, N, K, bits, words_per_row, chunk_offsets=None, chunk_cols=None,
                   chunk_vals=None, lora_H=None, lora_B=None, dora_gamma=None, lora_scale=1.0, group_size=0,
                   lora_A=None, prepared=None):
        return None


_register_ops()


def init_workspaces(max_N: int, max_K: int, device: torch.device) -> None:
    """Pre-size the split-K workspace so graph capture never allocates it
    (vllm_wlq/__init__.py:79-81)."""
    _C.init_workspaces(int(max_N), int(max_K), torch.device(device))


def check_workspaces(device) -> None:
    """Raise RuntimeError if a cross-block hand-off failed on a workspace of ``device``
    (the kernels then wrote the rows concerned, and every later call's rows, as NaN).
    Waits for the streams that used the workspaces; not for use inside graph capture."""
    _C.check_workspaces(torch.device(device))


def reset_workspaces(device) -> None:
    """Clear the counter area of every workspace of ``device`` (after check_workspaces
    raised and the calls that used them have finished)."""
    _C.reset_workspaces(torch.device(device))


def register() -> None:
    """vLLM general-plugin entry point (setup.py:47-51 of the reference); importing
    this package already registered the ops and the quantization config."""
    return None


from .quant_config import WLQFastShotConfig  # noqa: E402
from .linear_method import WLQLinearMethod  # noqa: E402

__all__ = ["WLQFastShotConfig", "WLQLinearMethod", "init_workspaces", "check_workspaces", "reset_workspaces",
           "register"]
