"""MI355X-native WLQ metalog-LUT quantized linear layer.

Package layout:

* ``libwlq_hip.so`` -- the C ABI (``include/wlq_abi.h``): gfx950 HIP kernels for
  the decode product, the prefill MFMA GEMM, bit-exact dequantization and the
  DoRA epilogue, plus host helpers for the load-time formats.
* ``vllm_wlq`` -- the vLLM plugin surface of the reference
  (``WLQFastShotConfig``, ``WLQLinearMethod``, ``torch.ops.wlq_fastShot.gemv`` /
  ``gemm`` and the ``_C`` extension), backed by the C ABI.
* ``formats`` / ``synth`` -- host-side layout helpers and the seeded synthetic
  layer generator used by tests and benchmarks.

There is no CPU fallback: importing ``vllm_wlq`` without the built extension
raises.
"""
from __future__ import annotations

import ctypes
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libwlq_hip.so")
ABI_HEADER = os.path.join(os.path.dirname(PKG_DIR), "include", "wlq_abi.h")

_abi = None


def load_abi() -> ctypes.CDLL:
    """Load ``libwlq_hip.so`` (import torch first in processes that use torch, so
    both share torch's HIP runtime)."""
    global _abi
    if _abi is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        _abi = ctypes.CDLL(LIB_PATH)
        _declare(_abi)
    return _abi


def _declare(lib: ctypes.CDLL) -> None:
    c_i32, c_i64, c_sz, c_f, vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float, ctypes.c_void_p
    sig = {
        "wlq_abi_version": (ctypes.c_int, []),
        "wlq_status_string": (ctypes.c_char_p, [ctypes.c_int]),
        "wlq_last_error": (ctypes.c_char_p, []),
        "wlq_words_per_row": (c_i64, [c_i64, c_i32]),
        "wlq_chunk_width": (c_i32, [c_i32]),
        "wlq_gemm_workspace_bytes": (c_sz, [c_i64, c_i64, c_i64, c_i32, c_i32, c_i32]),
        "wlq_gemv": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, c_f, c_i32, c_i64, c_i64, c_i32,
                                    c_i32, vp, c_sz, vp]),
        "wlq_gemm": (ctypes.c_int, [vp, vp, vp, vp, c_i64, c_i64, c_i64, c_i32, c_i64, c_i32, vp, vp, vp, vp, vp, vp,
                                    vp, c_f, c_i32, vp, c_sz, vp]),
        "wlq_prepared_bytes": (c_sz, [c_i64, c_i64, c_i32, c_i32, c_i64]),
        "wlq_prepare": (ctypes.c_int, [vp, vp, c_i64, c_i64, c_i32, c_i32, vp, vp, vp, c_i64, vp, c_sz, vp]),
        "wlq_gemm_prepared": (ctypes.c_int, [vp, vp, vp, vp, c_sz, vp, c_i64, c_i64, c_i64, c_i32, c_i64, c_i32, vp,
                                             vp, vp, c_i64, vp, vp, vp, vp, c_f, c_i32, vp, c_sz, vp]),
        "wlq_gemm_prepared_noalloc": (ctypes.c_int, [vp, vp, vp, vp, c_sz, vp, c_i64, c_i64, c_i64, c_i32, c_i64,
                                                     c_i32, vp, vp, vp, c_i64, vp, vp, vp, vp, c_f, c_i32, vp]),
        "wlq_dequant": (ctypes.c_int, [vp, vp, vp, c_i64, c_i64, c_i32, c_i64, c_i32, vp, vp, vp, vp]),
        "wlq_dora_epilogue": (ctypes.c_int, [vp, vp, vp, vp, c_f, c_i32, c_i64, c_i64, vp]),
        "wlq_workspace_status": (ctypes.c_int, [vp, c_sz, vp]),
        "wlq_workspace_reset": (ctypes.c_int, [vp, c_sz, vp]),
        "wlq_repack_row_aligned": (ctypes.c_int, [vp, c_i64, c_i64, c_i64, c_i32, vp, c_i64]),
        "wlq_ef_total": (c_i64, [vp, c_i64]),
        "wlq_ef_decode_chunk_csr": (ctypes.c_int, [vp, c_i64, vp, c_i64, c_i64, c_i64, c_i64, c_i64, vp, vp, c_i64,
                                                   ctypes.POINTER(c_i64)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


__all__ = ["PKG_DIR", "LIB_PATH", "ABI_HEADER", "load_abi"]
