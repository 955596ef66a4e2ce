"""Resource audit of every gfx950 kernel in the last build (CPU only).

rdnattention/_build.py records the compiler's kernel-resource-usage
remarks in build/kernel_resources.json.  This test holds the
kernels to what their launches assume (the reference audits its own tile
choices against a VGPR cap, tests/head_dim_resources.py):

* no register spills (scratch 0 bytes per lane);
* LDS per workgroup within gfx950's 160 KiB;
* enough occupancy for the waves one workgroup places on a SIMD (the
  8-wave kernels need 2 waves per SIMD, the 4-wave ones 1);
* every head dim the dispatchers can select is compiled in.
"""
import json
import os
import re

import pytest

from rdnattention import _build

LDS_LIMIT = 160 * 1024

# kernel name fragment -> waves of one workgroup per SIMD (workgroup waves / 4)
WAVES_PER_SIMD = {
    "fa_fwd_f16_pp": 2,
    "fa_fwd_int8": 2,
    "fa_fwd_int8_f16pv": 2,
    "fa_fwd_f16_kpair": 2,
    "fa_fwd_f16_dpair": 2,
    "fa_fwd_f16_decode": 1,
}


@pytest.fixture(scope="module")
def kernels():
    if not _build.RESOURCES.exists() or not _build.LIB.exists():
        _build.build()
    ks = json.loads(_build.RESOURCES.read_text())
    assert ks, "no kernel resources recorded"
    return ks


def _demangled_base(name):
    m = re.search(r"N_1\d+(\w+?)I", name) or re.search(r"N_1\d+(\w+?)E", name)
    return m.group(1) if m else name


def test_no_spills(kernels):
    spills = [(k["kernel"], k["scratch_bytes_per_lane"]) for k in kernels if k.get("scratch_bytes_per_lane", 0)]
    assert not spills, spills


def test_lds_within_gfx950_limit(kernels):
    over = [(k["kernel"], k["lds_bytes"]) for k in kernels if k["lds_bytes"] > LDS_LIMIT]
    assert not over, over


def test_occupancy_fits_the_workgroup(kernels):
    checked = 0
    for k in kernels:
        need = WAVES_PER_SIMD.get(_demangled_base(k["kernel"]))
        if need is not None:
            assert k["waves_per_simd"] >= need, (k["kernel"], k["waves_per_simd"], need)
            checked += 1
    # pp 4, kpair 4, dpair 8, decode 3, int8 3 + int8_f16pv 3 (+ 2 score-export instantiations)
    assert checked >= 4 + 4 + 3 + 5 + 3 + 4


def test_every_dispatched_head_dim_is_compiled(kernels):
    names = [k["kernel"] for k in kernels]

    def has(base, d):
        return any(f"{base}ILi{d}E" in n for n in names)

    for d in (32, 64, 96, 128):
        assert has("fa_fwd_f16_pp", d), d
    for d in (160, 192, 224, 256):
        assert has("fa_fwd_f16_kpair", d), d
    for d in range(288, 513, 32):
        assert has("fa_fwd_f16_dpair", d), d
    for d in (32, 64, 128):
        assert has("fa_fwd_f16_decode", d), d
    # INT8: head_dim 64 with both GEMMs on int8 MFMA, 128 (and the per-token V
    # scale) with P V on fp16 MFMA
    assert has("fa_fwd_int8", 64)
    for d in (64, 128):
        assert has("fa_fwd_int8_f16pv", d), d
    for frag in ("rope_rotate_rows", "fa_decode_combine", "quant_rows_kernel", "col_max_kernel",
                 "quant_cols_kernel"):
        assert any(frag in n for n in names), frag


ATTENTION_SOURCES = ["fa_fwd_f16.hip", "fa_fwd_f16_kpair.hip", "fa_fwd_f16_dpair.hip", "fa_fwd_int8.hip",
                     "fa_fwd_int8_f16pv.hip", "fa_fwd_decode.hip"]


def test_no_waterfall_loops(tmp_path):
    """A buffer descriptor that the compiler holds in vector registers (a
    wave-uniform value it cannot prove uniform) gets a loop around every load
    through it, once per distinct descriptor: v_readfirstlane of each dword,
    two v_cmp_eq_u64, an exec save and restore and a branch.  The D = 256
    wave-pair kernel had eight per key tile, 5 % of its time.  The attention
    kernels' device assembly, built with the library's flags, has none."""
    import shutil
    import subprocess

    if not shutil.which(_build.HIPCC) and not os.path.exists(_build.HIPCC):
        pytest.skip("hipcc not found")
    procs = []
    for src in ATTENTION_SOURCES:
        extra = ["-fno-honor-nans"] if src in _build.NO_NAN_SOURCES else []
        out = tmp_path / (src + ".s")
        cmd = [_build.HIPCC, "-x", "hip", "--offload-arch=gfx950", *_build.COMMON, *_build.DEVICE_FLAGS, *extra,
               "--cuda-device-only", "-S", str(_build.CSRC / src), "-o", str(out)]
        procs.append((src, out, subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.PIPE)))
    found = {}
    for src, out, p in procs:
        _, err = p.communicate(timeout=600)
        assert p.returncode == 0, (src, err.decode()[-2000:])
        n = sum(1 for line in out.read_text().splitlines() if "v_cmp_eq_u64" in line)
        if n:
            found[src] = n
    assert not found, found
