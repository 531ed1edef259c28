"""Packaging hook: compile libsol_attn_amd.so (hipcc, gfx950) before the package is collected.

The library is built in-tree by sol_attn_amd/_build.py, which recompiles every source on
each call, and ships as package data next to the Python layer that loads it.  Set
SOL_ATTN_AMD_PREBUILT=1 to package an already built library without recompiling.
Metadata lives in setup.cfg.
"""

import importlib.util
import os

from setuptools import setup
from setuptools.command.build_py import build_py
from setuptools.command.install import install
from setuptools.dist import Distribution

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "solattn-amd_amd", "sol_attn_amd")


class BuildHipLibrary(build_py):
    def run(self):
        lib = os.path.join(PKG, "libsol_attn_amd.so")
        if not (os.environ.get("SOL_ATTN_AMD_PREBUILT") == "1" and os.path.exists(lib)):
            # Load _build.py by path: importing the package would import torch, which an
            # isolated build environment does not have.
            spec = importlib.util.spec_from_file_location("sol_attn_amd_build", os.path.join(PKG, "_build.py"))
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            mod.build()
        super().run()


class BinaryDistribution(Distribution):
    """The package carries a native library, so it installs as a platform package."""

    def has_ext_modules(self):
        return True


class InstallPlatlib(install):
    """Install into platlib (distutils picks it only when ext_modules is non-empty)."""

    def finalize_options(self):
        super().finalize_options()
        self.install_lib = self.install_platlib


cmdclass = {"build_py": BuildHipLibrary, "install": InstallPlatlib}
try:
    from wheel.bdist_wheel import bdist_wheel

    class PlatformWheel(bdist_wheel):
        """Tag the wheel for the platform only: the gfx950 library is loaded with ctypes,
        so no Python ABI tag is needed."""

        def get_tag(self):
            return "py3", "none", super().get_tag()[2]

    cmdclass["bdist_wheel"] = PlatformWheel
except ImportError:
    pass

setup(distclass=BinaryDistribution, cmdclass=cmdclass)
