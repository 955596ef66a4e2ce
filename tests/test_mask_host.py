"""The kernels' mask helpers (rdnattention_amd/csrc/fa_mask.hpp), compiled for
the host and checked exhaustively: the per-row-tile class ranges that the
prefill kernels classify key tiles with equal classify_tile, which equals a
pair-by-pair evaluation of the reference's visibility rule
(src/rdna/fa2_forward_f16.hip:325-348)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_tile_classes_match_classify_tile(tmp_path):
    exe = tmp_path / "mask_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", f"-I{ROOT / 'rdnattention_amd' / 'csrc'}",
                    str(ROOT / "tests" / "cxx" / "mask_check.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok ")
    assert int(r.stdout.split()[1]) > 100000
