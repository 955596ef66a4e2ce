"""Wheel build: compiles librdnattention.so for gfx950 with hipcc
(rdnattention/_build.py) and places it in rdnattention/lib, the reference
wheel's layout (pyproject.toml:6, :66-67), so a wheel always carries the
library built from its own sources.

    pip wheel . --no-deps --no-build-isolation
"""
import importlib.util
import shutil
from pathlib import Path

from setuptools import setup
from setuptools.command.build_py import build_py
from setuptools.dist import Distribution

ROOT = Path(__file__).resolve().parent


class BinaryDistribution(Distribution):
    # the package carries a native library: a platform wheel, not a pure one
    def has_ext_modules(self):
        return True


class BuildWithLibrary(build_py):
    def run(self):
        # load the build module by path: importing the package is not needed
        # (and would import the runtime wrapper) to compile the library
        spec = importlib.util.spec_from_file_location("rdnattention_build", ROOT / "rdnattention" / "_build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        lib = mod.build()
        dest = ROOT / "rdnattention" / "lib"
        dest.mkdir(exist_ok=True)
        shutil.copy2(lib, dest / lib.name)
        super().run()


setup(
    name="rdnattention",
    version="0.1.0",
    description="FlashAttention-2 forward for AMD MI355X (gfx950): a drop-in for RDNAttention's attention path",
    long_description=(ROOT / "README.md").read_text(),
    long_description_content_type="text/markdown",
    python_requires=">=3.9",
    # the wrapper takes torch (ROCm) tensors; torch is not pinned, as in the
    # reference (pyproject.toml:39-49)
    install_requires=[],
    packages=["rdnattention"],
    package_data={"rdnattention": ["lib/librdnattention.so"]},
    cmdclass={"build_py": BuildWithLibrary},
    distclass=BinaryDistribution,
)
