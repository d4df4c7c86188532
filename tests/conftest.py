import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# The library reads WLQ_TEST_HOOKS once, at its first product: on for the whole test process, so
# a test may set a hook's variable (WLQ_TEST_FORCE_PREFILL, ...) for its own calls.  With none of
# them set the products run exactly as without the hooks.
os.environ.setdefault("WLQ_TEST_HOOKS", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def vw():
    """The plugin package (imports torch first so the C ABI shares torch's HIP runtime)."""
    import torch  # noqa: F401

    import qwen_wlqfastshot_helen_beta_amd.vllm_wlq as m

    return m
