"""``vllm_wlq``: the reference's import name for the plugin package.

``import vllm_wlq`` (what vLLM's ``vllm.general_plugins`` entry point
``vllm_wlq = vllm_wlq:register`` does, and what the reference's users write)
returns ``qwen_wlqfastshot_helen_beta_amd.vllm_wlq`` itself, and
``vllm_wlq.<submodule>`` its submodules, so both names share one set of module
objects: the torch ops, the registered ``wlq_fastShot`` config and the
``_C`` extension are registered once.
"""
import importlib
import sys

_REAL = "qwen_wlqfastshot_helen_beta_amd.vllm_wlq"
_SUBMODULES = ("_C", "_vllm_compat", "quant_config", "linear_method")

_pkg = importlib.import_module(_REAL)
for _name in _SUBMODULES:
    sys.modules[f"{__name__}.{_name}"] = importlib.import_module(f"{_REAL}.{_name}")
sys.modules[__name__] = _pkg
