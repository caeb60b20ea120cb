"""Setuptools shim: the metadata and the vLLM plugin entry point live in setup.cfg.

    pip install --no-build-isolation ./amass-kv_amd     # builds libamass_hip.so if absent

build_py compiles the HIP library (build_hip.py, hipcc --offload-arch=gfx950) when
amass/_lib/libamass_hip.so is missing, so the wheel always carries it as package data.
"""
import os
import sys

from setuptools import Distribution, setup
from setuptools.command.build_py import build_py

HERE = os.path.dirname(os.path.abspath(__file__))


class BuildWithHip(build_py):
    def run(self):
        if not os.path.exists(os.path.join(HERE, "amass", "_lib", "libamass_hip.so")):
            sys.path.insert(0, HERE)
            import build_hip
            build_hip.build()
            build_hip.build_calib()
        super().run()


class BinaryDistribution(Distribution):
    """The wheel carries a gfx950 shared library, so it is tagged for this platform."""

    def has_ext_modules(self):
        return True


setup(cmdclass={"build_py": BuildWithHip}, distclass=BinaryDistribution)
