"""setuptools entry of the fable_attn distribution (metadata in setup.cfg).

Building the wheel compiles the HIP library first when it is absent (build.py: hipcc for gfx950
over csrc/*.hip, headers from ../include), or always with FABLE_ATTN_REBUILD=1, and ships it as
package data; the wheel is therefore platform-specific (linux, gfx950 code objects inside).
"""
import os
import subprocess
import sys

from setuptools import setup
from setuptools.command.build_py import build_py
from setuptools.dist import Distribution

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "fable_attn", "libfable_attn_hip.so")


class BuildPyWithLibrary(build_py):
    def run(self):
        if not os.path.exists(LIB) or os.environ.get("FABLE_ATTN_REBUILD"):
            subprocess.run([sys.executable, os.path.join(HERE, "build.py")], check=True)
        super().run()


class BinaryDistribution(Distribution):
    """A wheel that carries a native library is not pure Python."""

    def has_ext_modules(self):
        return True


setup(cmdclass={"build_py": BuildPyWithLibrary}, distclass=BinaryDistribution)
