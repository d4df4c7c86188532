"""Build and install the vllm_wlq plugin (metadata and entry point in setup.cfg).

``pip install --no-build-isolation .`` compiles libwlq_hip.so (hipcc, gfx950) and
the torch extension ``_C`` in the source tree first (``_build.build_all``), then
installs them as package data; torch must already be installed (ROCm build).
"""
from setuptools import setup
from setuptools.command.build_py import build_py


class BuildNative(build_py):
    """build_py that compiles the native parts before copying the package files."""

    def run(self):
        from qwen_wlqfastshot_helen_beta_amd import _build

        _build.build_all()
        super().run()


setup(cmdclass={"build_py": BuildNative})
