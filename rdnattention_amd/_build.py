"""Builds librdnattention.so for gfx950 with hipcc (no cmake, no JIT cache).

    python -m rdnattention_amd._build [--arch gfx950] [--no-int8] [-v]

Objects go to rdnattention_amd/_build/, the library to
rdnattention_amd/lib/librdnattention.so (in-tree, so it travels with the
repository snapshot to the GPU machine).  Mirrors the reference's build
options (CMakeLists.txt:3-5 forced Release, :33 RDNATTENTION_ENABLE_INT8)
for one architecture, gfx950.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "librdnattention.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in device code (the host pass
# warns that it does not know the feature; harmless).
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", f"-I{ROOT / 'include'}"]


def sources():
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path, arch: str, defines, verbose: bool) -> Path:
    out = OBJ / (src.name + ".o")
    if src.suffix == ".hip":
        cmd = [HIPCC, "-x", "hip", f"--offload-arch={arch}", *COMMON, *DEVICE_FLAGS, *defines, "-c", str(src),
               "-o", str(out)]
    else:
        cmd = [HIPCC, "-x", "c++", *COMMON, "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", *defines, "-c",
               str(src), "-o", str(out)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
    if verbose and r.stderr.strip():
        lines = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln]
        if lines:
            print("\n".join(lines), file=sys.stderr)
    return out


def build(arch: str = "gfx950", int8: bool = True, verbose: bool = False, jobs: int | None = None) -> Path:
    OBJ.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    defines = [] if int8 else ["-DRDNATTENTION_NO_INT8"]
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, arch, defines, verbose), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={arch}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    shutil.move(str(tmp), str(LIB))
    return LIB


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--arch", default="gfx950")
    ap.add_argument("--no-int8", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args(argv)
    path = build(args.arch, not args.no_int8, args.verbose)
    print(path)


if __name__ == "__main__":
    main()
