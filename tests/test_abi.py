"""CPU-side checks of the C ABI boundary (no GPU needed):

* librdnattention.so loads and exports every symbol declared in include/*.h
  (the four drop-in symbols of the reference's src/c_api.hpp:16-87 plus the
  extensions in rdnattention_ext.h) and the reference's C++ launch API;
* every argument check runs before any HIP call and reports -3 with the
  reference's message format ("Attention (fp16) failed: ...");
* the Python wrapper raises the reference's exception types for bad input.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "build" / "librdnattention.so"


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        from rdnattention import _build

        _build.build()
    import rdnattention

    return rdnattention._lib_handle()


def _declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        names.update(re.findall(r"RDNA_API\s+[\w\s\*]+?\b(rdna_\w+)\s*\(", text))
    return names


def test_exports_every_declared_symbol(lib):
    declared = _declared_symbols()
    assert {"rdna_has_device", "rdna_get_error", "rdna_attention_forward",
            "rdna_attention_forward_int8qk"} <= declared
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s+(\S+)", out))
    missing = declared - exported
    assert not missing, f"declared but not exported: {missing}"
    # the reference's C++ API (src/rdna/fa2_forward_f16.hpp, fa2_forward_int8qk.hpp)
    for mangled in ("_ZN4rdna10forwardF16ERKNS_13ForwardParamsEPv", "_ZN4rdna9lastErrorEv", "_ZN4rdna9hasDeviceEv",
                    "_ZN4rdna13forwardInt8QKERKNS_19ForwardParamsInt8QKEPv", "_ZN4rdna15lastErrorInt8QKEv"):
        assert mangled in exported


def test_version(lib):
    assert lib.rdna_version().decode().startswith("0.1.0")


def _buf(n=4096):
    # 16-byte aligned host buffer; never dereferenced by the rejected calls below
    a = np.zeros(n + 16, dtype=np.uint8)
    off = (-a.ctypes.data) % 16
    return a, a.ctypes.data + off


def _fwd(lib, **kw):
    hold, p = _buf()
    args = dict(q=p, k=p, v=p, o=p, cos=None, sin=None, strides=(64 * 8 * 64, 8 * 64, 64), B=1, Hq=8, Hkv=8, Sq=8,
                Sk=8, D=64, scale=0.125, causal=0, rope=0, window=-1)
    args.update(kw)
    s = args["strides"]
    rc = lib.rdna_attention_forward(args["q"], args["k"], args["v"], args["o"], args["cos"], args["sin"],
                                    *s, *s, *s, *s, args["B"], args["Hq"], args["Hkv"], args["Sq"], args["Sk"],
                                    args["D"], args["scale"], args["causal"], args["rope"], args["window"], None)
    return rc, lib.rdna_get_error().decode()


@pytest.mark.parametrize("kw,msg", [
    (dict(D=48), "unsupported head_dim (multiples of 32 from 32 to 512)"),
    (dict(D=544), "unsupported head_dim"),
    (dict(D=0), "unsupported head_dim"),
    (dict(Hkv=3), "numHeads must be a positive multiple of numKvHeads"),
    (dict(Hkv=0), "numHeads must be a positive multiple of numKvHeads"),
    (dict(Sq=0), "empty launch grid"),
    (dict(B=0), "empty launch grid"),
    (dict(q=None), "null tensor pointer"),
    (dict(strides=(4096, 512, 68)), "multiples of 16 bytes"),
    (dict(rope=1), "rot_cos/rot_sin is null"),
    (dict(Sq=(1 << 30) + 1), "exceed the supported range"),
])
def test_fp16_argument_errors(lib, kw, msg):
    rc, err = _fwd(lib, **kw)
    assert rc == -3
    assert err.startswith("Attention (fp16) failed: ")
    assert msg in err


def test_misaligned_pointer_rejected(lib):
    hold, p = _buf()
    rc, err = _fwd(lib, q=p + 2)
    assert rc == -3 and "16-byte aligned" in err


def test_error_is_thread_local_and_sticky(lib):
    import threading

    _fwd(lib, D=48)
    seen = {}

    def other():
        seen["err"] = lib.rdna_get_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["err"] == ""  # a fresh thread has no error
    assert "head_dim" in lib.rdna_get_error().decode()  # not cleared


def _i8(lib, **kw):
    hold, p = _buf()
    args = dict(B=1, Hq=8, Hkv=8, Sq=8, Sk=8, D=64, strides=(8 * 8 * 64, 8 * 64, 64))
    args.update(kw)
    s = args["strides"]
    rc = lib.rdna_attention_forward_int8qk(p, p, p, p, *s, *s, *s, *s, args["B"], args["Hq"], args["Hkv"],
                                           args["Sq"], args["Sk"], args["D"], 0.125, 1.0, 1.0, 1.0, None, None, 0,
                                           -1, None)
    return rc, lib.rdna_get_error().decode()


@pytest.mark.parametrize("kw,msg", [
    (dict(D=96), "unsupported head_dim (only 64 and 128 are compiled in for the int8 kernel)"),
    (dict(Hkv=0), "numHeads must be a positive multiple of numKvHeads"),
    (dict(Hkv=3, D=96), "numHeads must be a positive multiple of numKvHeads"),  # ratio checked first
    (dict(strides=(4096, 512, 72)), "multiples of 16 bytes"),
])
def test_int8_argument_errors(lib, kw, msg):
    rc, err = _i8(lib, **kw)
    assert rc == -3
    assert err.startswith("Attention (int8qk) failed: ")
    assert msg in err


def test_int8_vtoken_argument_errors(lib):
    """rdna_attention_forward_int8qk_vtoken: the scale array is required, 4-byte
    aligned, and checked before any HIP call."""
    import rdnattention

    rdnattention._lib_handle()
    hold, p = _buf()
    s = (8 * 8 * 64, 8 * 64, 64)

    def call(vt):
        rc = lib.rdna_attention_forward_int8qk_vtoken(p, p, p, p, *s, *s, *s, *s, 1, 8, 8, 8, 8, 64, 0.125, 1.0,
                                                      1.0, 1.0, None, None, vt, 0, -1, None)
        return rc, lib.rdna_get_error().decode()

    rc, err = call(None)
    assert rc == -3 and "v_token_vec is null" in err
    rc, err = call(p + 2)
    assert rc == -3 and "v_token_vec must be a 4-byte aligned" in err


def test_has_device_without_gpu(lib):
    import torch

    if torch.cuda.is_available():
        pytest.skip("GPU host")
    assert lib.rdna_has_device() == 0


# --------------------------------------------------------------------------- #
# Python wrapper argument checks (rdnattention/__init__.py:138-192)
# --------------------------------------------------------------------------- #
def test_python_type_errors():
    import torch

    import rdnattention as ra

    with pytest.raises(TypeError):
        ra.flash_attn(np.zeros((1, 1, 1, 64)), None, None)
    cpu = torch.zeros(1, 2, 4, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="must be on a HIP device"):
        ra.flash_attn(cpu, cpu, cpu)


def test_python_head_dim_lists():
    import rdnattention as ra

    assert ra.SUPPORTED_HEAD_DIMS == tuple(range(32, 513, 32))
    assert ra.SUPPORTED_HEAD_DIMS_INT8 == (64, 128)
    with pytest.raises(ra.RDNAttentionError, match="head_dim 48 not supported"):
        ra._check_head_dim(48, "flash_attn")
    assert set(ra.__all__) == {"flash_attn", "flash_attn_int8qk", "flash_attn_int8qk_quantized",
                               "quantize_int8_perchannel_v", "quantize_int8_qk_pertoken", "has_device",
                               "RDNAttentionError", "SUPPORTED_HEAD_DIMS", "SUPPORTED_HEAD_DIMS_INT8",
                               "__version__"}


def test_python_missing_library(monkeypatch, tmp_path):
    import rdnattention as ra

    monkeypatch.setenv("RDNATTENTION_LIB", str(tmp_path / "nope.so"))
    monkeypatch.setattr(ra, "_lib", None)
    with pytest.raises(ra.RDNAttentionError, match="missing file"):
        ra.has_device()


def test_kernel_timer_without_launches(lib):
    """Enable/read of the kernel timer with nothing launched: no HIP call is
    made, zero launches are reported, the record is cleared."""
    import ctypes

    lib.rdna_kernel_timer_enable.argtypes = [ctypes.c_int32]
    lib.rdna_kernel_timer_read.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)]
    assert lib.rdna_kernel_timer_enable(1) == 0
    ms, n = ctypes.c_double(-1.0), ctypes.c_int64(-1)
    assert lib.rdna_kernel_timer_read(ctypes.byref(ms), ctypes.byref(n)) == 0
    assert ms.value == 0.0 and n.value == 0
    assert lib.rdna_kernel_timer_read(None, None) == -3
    assert lib.rdna_kernel_timer_enable(0) == 0


def _quant(lib, **kw):
    hold, p = _buf()
    args = dict(x=p, dtype=0, strides=(8 * 16 * 64, 16 * 64, 64), B=1, H=8, S=16, D=64, per_channel=0, cos=None,
                sin=None, q=p, sc=p)
    args.update(kw)
    s = args["strides"]
    rc = lib.rdna_quantize_int8(args["x"], args["dtype"], *s, args["B"], args["H"], args["S"], args["D"],
                                args["per_channel"], args["cos"], args["sin"], args["q"], args["sc"], None)
    return rc, lib.rdna_get_error().decode()


@pytest.mark.parametrize("kw,msg", [
    (dict(D=12), "head_dim must be a multiple of 8 from 8 to 512"),
    (dict(D=520), "head_dim must be a multiple of 8 from 8 to 512"),
    (dict(dtype=2), "x_dtype must be 0 (fp16) or 1 (fp32)"),
    (dict(S=0), "empty tensor"),
    (dict(x=None), "null tensor pointer"),
    (dict(strides=(8192, 1024, 68)), "strides of x must be multiples of 16 bytes"),
    (dict(dtype=1, strides=(8192, 1024, 66)), "strides of x must be multiples of 16 bytes"),
    (dict(cos="p"), "pass both rot_cos and rot_sin, or neither"),
    (dict(cos="p", sin="p", per_channel=1), "RoPE applies to the per-token scheme only"),
    (dict(cos="p+4", sin="p"), "rot_cos and rot_sin must be 16-byte aligned"),
])
def test_quantize_argument_errors(lib, kw, msg):
    hold, p = _buf()
    kw = {k: (p if v == "p" else p + 4 if v == "p+4" else v) for k, v in kw.items()}
    rc, err = _quant(lib, **kw)
    assert rc == -3
    assert err.startswith("Quantize (int8) failed: ")
    assert msg in err


def test_int8_vchannel_misaligned_rejected(lib):
    hold, p = _buf()
    s = (8 * 8 * 64, 8 * 64, 64)
    rc = lib.rdna_attention_forward_int8qk_vchannel(p, p, p, p, *s, *s, *s, *s, 1, 8, 8, 8, 8, 64, 0.125, 1.0, 1.0,
                                                     1.0, None, None, p + 4, 0, -1, None)
    assert rc == -3
    assert "v_channel_vec must be a 16-byte aligned float array" in lib.rdna_get_error().decode()


def test_pertoken_rope_cpu_path_matches_oracle():
    """quantize_int8_qk_pertoken on CPU tensors with RoPE tables: the torch
    rotation equals the oracle's (fp32 products, fp16 rounding) and the rows
    are then quantised by the reference formulas."""
    import numpy as np
    import torch

    import oracle
    import rdnattention as ra

    g = torch.Generator().manual_seed(17)
    q = torch.randn(1, 2, 40, 64, generator=g).half()
    k = torch.randn(1, 2, 40, 64, generator=g).half()
    cos, sin = oracle.rope_tables(40, 64)
    qi, ki, qs, ks = ra.quantize_int8_qk_pertoken(q, k, rot_cos=torch.from_numpy(cos), rot_sin=torch.from_numpy(sin))
    for x, xi, xs in ((q, qi, qs), (k, ki, ks)):
        rot = oracle.rope(x.float().numpy(), cos, sin, round_f16=True)
        assert np.array_equal(ra._rope_torch(x, torch.from_numpy(cos), torch.from_numpy(sin)).float().numpy(), rot)
        ri, rs = oracle.quant_pertoken(rot)
        assert np.array_equal(xi.numpy(), ri) and np.allclose(xs.numpy(), rs, rtol=1e-6, atol=0)
    with pytest.raises(ValueError, match="both"):
        ra.quantize_int8_qk_pertoken(q, k, rot_cos=torch.from_numpy(cos))


def test_pertoken_v_cpu_path_matches_oracle():
    """quantize_int8_pertoken_v on a CPU tensor: the per-token formula of
    quantize_int8_qk_pertoken (rdnattention/__init__.py:335-339), as the
    oracle's quantiser computes it."""
    import numpy as np
    import torch

    import oracle
    import rdnattention as ra

    g = torch.Generator().manual_seed(18)
    v = torch.randn(2, 3, 50, 64, generator=g).half()
    v[0, 0, 3] = 0  # an all-zero row: scale 1
    vi, vt = ra.quantize_int8_pertoken_v(v)
    ri, rs = oracle.quant_pertoken(v.float().numpy())
    assert vi.dtype == torch.int8 and vt.shape == (2, 3, 50) and vt.is_contiguous()
    assert np.array_equal(vi.numpy(), ri) and np.allclose(vt.numpy(), rs, rtol=1e-6, atol=0)
    assert vt[0, 0, 3].item() == 1.0


def test_scratch_trim_without_pools(lib):
    """rdna_scratch_trim with no pool created yet (no HIP call made) is a no-op."""
    lib.rdna_scratch_trim.restype = ctypes.c_int32
    assert lib.rdna_scratch_trim() == 0


def test_scratch_stats_without_device(lib):
    """rdna_scratch_stats of a device the library never used reports nothing
    cached and no allocator call; a null output pointer is refused with -3."""
    lib.rdna_scratch_stats.restype = ctypes.c_int32
    lib.rdna_scratch_stats.argtypes = [ctypes.c_int32, ctypes.POINTER(ctypes.c_uint64),
                                       ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]
    nbytes, entries, allocs = ctypes.c_uint64(7), ctypes.c_int64(7), ctypes.c_int64(7)
    assert lib.rdna_scratch_stats(0, ctypes.byref(nbytes), ctypes.byref(entries), ctypes.byref(allocs)) == 0
    assert (nbytes.value, entries.value, allocs.value) == (0, 0, 0)
    assert lib.rdna_scratch_stats(0, None, ctypes.byref(entries), ctypes.byref(allocs)) == -3
    lib.rdna_get_error.restype = ctypes.c_char_p
    assert b"null output pointer" in lib.rdna_get_error()
