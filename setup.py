"""Wheel build: compiles librdnattention.so for gfx950 with hipcc into
rdnattention_amd/lib (rdnattention_amd/_build.py) before packaging it, so a
wheel always carries the library built from its own sources.

    pip wheel . --no-deps --no-build-isolation
"""
import importlib.util
from pathlib import Path

from setuptools import setup
from setuptools.command.build_py import build_py
from setuptools.dist import Distribution


class BinaryDistribution(Distribution):
    # the package carries a native library: a platform wheel, not a pure one
    def has_ext_modules(self):
        return True


class BuildWithLibrary(build_py):
    def run(self):
        # load the build module by path: importing the package is not needed
        # (and would import the runtime wrapper) to compile the library
        path = Path(__file__).resolve().parent / "rdnattention_amd" / "_build.py"
        spec = importlib.util.spec_from_file_location("rdnattention_amd_build", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
        super().run()


setup(
    name="rdnattention-amd",
    version="0.1.0",
    description="FlashAttention-2 forward for AMD MI355X (gfx950): a drop-in for RDNAttention's attention path",
    long_description=(Path(__file__).resolve().parent / "README.md").read_text(),
    long_description_content_type="text/markdown",
    python_requires=">=3.9",
    # the wrapper takes torch (ROCm) tensors; torch is not pinned, as in the
    # reference (pyproject.toml:39-49)
    install_requires=["numpy"],
    packages=["rdnattention_amd"],
    # the library sits in the package's lib/ directory, as in the reference's
    # wheel (rdnattention/lib, pyproject.toml:66-67)
    package_data={"rdnattention_amd": ["lib/librdnattention.so", "csrc/*.hip", "csrc/*.hpp", "csrc/*.cpp"]},
    cmdclass={"build_py": BuildWithLibrary},
    distclass=BinaryDistribution,
)
