"""Builds librdnattention.so for gfx950 with hipcc (no cmake, no JIT cache).

    python -m rdnattention._build [--arch gfx950] [--no-int8] [--out DIR] [-v]

Sources are rdnattention_amd/csrc/*.{hip,cpp}.  Objects go to build/obj/,
the library to build/librdnattention.so -- the development build that the
package prefers in a source checkout, as the reference's wrapper prefers its
CMake build/ directory (rdnattention/__init__.py:55-61) -- and the
compiler's per-kernel resource usage to build/kernel_resources.json.  The
wheel (setup.py) copies the library into rdnattention/lib/.  Mirrors the
reference's build options (CMakeLists.txt:3-5 forced Release, :33
RDNATTENTION_ENABLE_INT8) for one architecture, gfx950.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import json
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = ROOT / "rdnattention_amd" / "csrc"
BUILD = ROOT / "build"
LIB_NAME = "librdnattention.so"
LIB = BUILD / LIB_NAME
# per-kernel resource usage of the last build (VGPRs, AGPRs, scratch, LDS,
# occupancy), from the compiler's kernel-resource-usage remarks
RESOURCES = BUILD / "kernel_resources.json"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in device code (the host pass
# warns that it does not know the feature; harmless).
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# FP16 attention kernels: their row maxima (fmaxf over MFMA results and lane
# exchanges) otherwise get a canonicalising v_max per input that is not known
# to be a quiet NaN; scores are never NaN there (masked scores are -inf, and
# every -inf - -inf case is selected away), so the five extra VALU per tile
# are dropped.  Infinities keep IEEE semantics.  The quantisers keep the
# default: their amax must treat NaN inputs as torch does.
NO_NAN_SOURCES = {"fa_fwd_f16.hip", "fa_fwd_f16_kpair.hip", "fa_fwd_f16_dpair.hip", "fa_fwd_int8.hip",
                  "fa_fwd_int8_f16pv.hip"}
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", f"-I{ROOT / 'include'}"]


def sources():
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]"
                     r"|LDS Size \[bytes/block\]|TotalSGPRs): (\S+)")
_KEYS = {"VGPRs": "vgprs", "AGPRs": "agprs", "ScratchSize [bytes/lane]": "scratch_bytes_per_lane",
         "Occupancy [waves/SIMD]": "waves_per_simd", "LDS Size [bytes/block]": "lds_bytes", "TotalSGPRs": "sgprs"}


def parse_resource_remarks(text: str, source: str):
    """Kernel-resource-usage remarks -> [{"kernel", "source", "vgprs", ...}]."""
    kernels = []
    for m in _REMARK.finditer(text):
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            kernels.append({"kernel": val, "source": source})
        elif kernels:
            kernels[-1][_KEYS[key]] = int(val)
    return kernels


def _compile(src: Path, obj_dir: Path, arch: str, defines, verbose: bool):
    out = obj_dir / (src.name + ".o")
    if src.suffix == ".hip":
        extra = ["-fno-honor-nans"] if src.name in NO_NAN_SOURCES else []
        cmd = [HIPCC, "-x", "hip", f"--offload-arch={arch}", *COMMON, *DEVICE_FLAGS, *extra, *defines,
               "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(out)]
    else:
        cmd = [HIPCC, "-x", "c++", *COMMON, "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", *defines, "-c",
               str(src), "-o", str(out)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
    if verbose and r.stderr.strip():
        lines = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln and "remark:" not in ln]
        if lines:
            print("\n".join(lines), file=sys.stderr)
    return out, parse_resource_remarks(r.stderr, src.name)


def build(arch: str = "gfx950", int8: bool = True, verbose: bool = False, jobs: int | None = None,
          out_dir: Path | None = None) -> Path:
    """Compile and link; returns the library path (out_dir/librdnattention.so,
    default build/).  int8=False is the reference's RDNATTENTION_ENABLE_INT8=OFF
    build: the INT8 entry points stay exported and return -4."""
    out_dir = Path(out_dir) if out_dir is not None else BUILD
    obj_dir = out_dir / ("obj" if int8 else "obj_noint8")
    obj_dir.mkdir(parents=True, exist_ok=True)
    lib = out_dir / LIB_NAME
    defines = [] if int8 else ["-DRDNATTENTION_NO_INT8"]
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(lambda s: _compile(s, obj_dir, arch, defines, verbose), srcs))
    objs = [o for o, _ in results]
    (out_dir / RESOURCES.name).write_text(json.dumps([k for _, ks in results for k in ks], indent=1))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={arch}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    shutil.move(str(tmp), str(lib))
    return lib


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--arch", default="gfx950")
    ap.add_argument("--no-int8", action="store_true")
    ap.add_argument("--out", type=Path, default=None, help="output directory (default: build/)")
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args(argv)
    path = build(args.arch, not args.no_int8, args.verbose, out_dir=args.out)
    print(path)


if __name__ == "__main__":
    main()
