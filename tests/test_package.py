"""The Python package under the reference's name and its build options (CPU only).

* ``import rdnattention`` gives the reference's public names
  (rdnattention/__init__.py:360-363) and its library search order
  (rdnattention/__init__.py:37-73): RDNATTENTION_LIB, then the development
  build build/ before the packaged lib/ in a source checkout, lib/ first
  otherwise;
* the shape checks that stand between a caller and an out-of-bounds kernel
  read raise ValueError before any library call;
* the INT8-disabled build (the reference's RDNATTENTION_ENABLE_INT8=OFF,
  CMakeLists.txt:33) keeps every INT8 symbol exported and returns -4 with the
  "Attention (int8qk) unavailable: ..." text (src/c_api.cpp:115-154), without
  touching a GPU.
"""
import ctypes
import importlib.util
import shutil
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
REFERENCE_ALL = ["flash_attn", "flash_attn_int8qk", "flash_attn_int8qk_quantized", "quantize_int8_perchannel_v",
                 "quantize_int8_qk_pertoken", "has_device", "RDNAttentionError", "SUPPORTED_HEAD_DIMS",
                 "SUPPORTED_HEAD_DIMS_INT8", "__version__"]


def test_public_names():
    import rdnattention

    assert rdnattention.__all__ == REFERENCE_ALL
    for name in REFERENCE_ALL:
        assert hasattr(rdnattention, name), name
    assert rdnattention.SUPPORTED_HEAD_DIMS == tuple(range(32, 513, 32))
    assert rdnattention.SUPPORTED_HEAD_DIMS_INT8 == (64, 128)
    assert issubclass(rdnattention.RDNAttentionError, Exception)


def _load_copy(tmp_path, source_tree: bool):
    """The package's __init__.py installed under tmp_path/<site>/rdnattention,
    optionally next to an rdnattention_amd/csrc directory (a source checkout),
    with both candidate libraries present as placeholder files."""
    site = tmp_path / ("src" if source_tree else "site")
    pkg = site / "rdnattention"
    (pkg / "lib").mkdir(parents=True)
    shutil.copy(ROOT / "rdnattention" / "__init__.py", pkg / "__init__.py")
    (pkg / "lib" / "librdnattention.so").write_bytes(b"")
    (site / "build").mkdir()
    (site / "build" / "librdnattention.so").write_bytes(b"")
    if source_tree:
        (site / "rdnattention_amd" / "csrc").mkdir(parents=True)
    name = f"rdnattention_copy_{int(source_tree)}"
    spec = importlib.util.spec_from_file_location(name, pkg / "__init__.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod, site


@pytest.mark.parametrize("source_tree", [True, False])
def test_library_search_order(tmp_path, monkeypatch, source_tree):
    monkeypatch.delenv("RDNATTENTION_LIB", raising=False)
    mod, site = _load_copy(tmp_path, source_tree)
    dev = site / "build" / "librdnattention.so"
    packaged = site / "rdnattention" / "lib" / "librdnattention.so"
    want = [dev, packaged] if source_tree else [packaged, dev]
    assert mod._library_candidates() == want
    assert mod._find_library() == want[0]
    want[0].unlink()
    assert mod._find_library() == want[1]
    want[1].unlink()
    with pytest.raises(mod.RDNAttentionError, match="Searched"):
        mod._find_library()


def test_library_override(tmp_path, monkeypatch):
    mod, _ = _load_copy(tmp_path, True)
    lib = tmp_path / "elsewhere.so"
    lib.write_bytes(b"")
    monkeypatch.setenv("RDNATTENTION_LIB", str(lib))
    assert mod._find_library() == lib
    monkeypatch.setenv("RDNATTENTION_LIB", str(tmp_path / "missing.so"))
    with pytest.raises(mod.RDNAttentionError, match="missing file"):
        mod._find_library()


def test_in_repo_library_is_the_build(monkeypatch):
    """In this checkout the package loads build/librdnattention.so."""
    import rdnattention

    monkeypatch.delenv("RDNATTENTION_LIB", raising=False)
    assert rdnattention._find_library() == ROOT / "build" / "librdnattention.so"


@pytest.mark.parametrize("q,k,v,msg", [
    ((2, 8, 64, 64), (1, 2, 64, 64), (1, 2, 64, 64), "Batch size"),
    ((2, 8, 64, 64), (2, 2, 64, 64), (2, 2, 32, 64), "same shape"),
    ((2, 8, 64, 64), (2, 2, 64, 64), (2, 4, 64, 64), "same shape"),
    ((2, 8, 64, 64), (2, 2, 64, 32), (2, 2, 64, 32), "head_dim"),
    ((2, 8, 64, 64), (2, 3, 64, 64), (2, 3, 64, 64), "multiple"),
])
def test_shape_checks(q, k, v, msg):
    """Each mismatch that would let a kernel read past a smaller K/V is a
    ValueError (the shapes are checked, not the data: CPU tensors suffice)."""
    import torch

    import rdnattention

    with pytest.raises(ValueError, match=msg):
        rdnattention._check_shapes(torch.empty(q), torch.empty(k), torch.empty(v))


def test_shape_checks_accept():
    import torch

    import rdnattention

    # GQA, cross-attention (Sk != Sq), MQA
    for q, kv in (((2, 8, 64, 64), (2, 2, 64, 64)), ((1, 4, 3, 128), (1, 4, 900, 128)), ((1, 8, 5, 32), (1, 1, 7, 32))):
        rdnattention._check_shapes(torch.empty(q), torch.empty(kv), torch.empty(kv))


@pytest.fixture(scope="module")
def noint8_lib(tmp_path_factory):
    sys.path.insert(0, str(ROOT))
    from rdnattention import _build

    out = tmp_path_factory.mktemp("noint8")
    path = _build.build(int8=False, out_dir=out)
    return ctypes.CDLL(str(path))


def _int8_args(extra_ptr: bool):
    vp = [None] * 4
    strides = [0] * 12
    dims = [1, 1, 1, 16, 16, 64]
    scales = [0.125, 1.0, 1.0, 1.0]
    vecs = [None, None] + ([None] if extra_ptr else [])
    return vp + strides + dims + scales + vecs + [0, -1, None]


def test_no_int8_build_returns_minus_4(noint8_lib):
    L = noint8_lib
    L.rdna_get_error.restype = ctypes.c_char_p
    I64, U32, F32, I32, VP = ctypes.c_int64, ctypes.c_uint32, ctypes.c_float, ctypes.c_int32, ctypes.c_void_p
    base = [VP] * 4 + [I64] * 12 + [U32] * 6 + [F32] * 4 + [VP, VP]
    tail = [I32, I32, VP]
    L.rdna_attention_forward_int8qk.argtypes = base + tail
    L.rdna_attention_forward_int8qk_vchannel.argtypes = base + [VP] + tail
    L.rdna_attention_forward_int8qk_vtoken.argtypes = base + [VP] + tail
    for fn, extra in ((L.rdna_attention_forward_int8qk, False), (L.rdna_attention_forward_int8qk_vchannel, True),
                      (L.rdna_attention_forward_int8qk_vtoken, True)):
        fn.restype = I32
        assert fn(*_int8_args(extra)) == -4
        err = L.rdna_get_error().decode()
        assert err.startswith("Attention (int8qk) unavailable: ") and "rdna_attention_forward()" in err, err
    L.rdna_int8_qk_scores.argtypes = [VP] * 3 + [I64] * 6 + [U32] * 6 + [VP]
    L.rdna_int8_qk_scores.restype = I32
    assert L.rdna_int8_qk_scores(None, None, None, 0, 0, 0, 0, 0, 0, 1, 1, 1, 16, 16, 64, None) == -4


def test_no_int8_build_exports_and_kernels(noint8_lib):
    """The INT8 symbols stay in the ABI; no INT8 kernel is compiled in."""
    path = Path(noint8_lib._name)
    for sym in ("rdna_attention_forward", "rdna_attention_forward_int8qk", "rdna_attention_forward_int8qk_vchannel",
                "rdna_attention_forward_int8qk_vtoken", "rdna_get_error", "rdna_has_device"):
        assert hasattr(noint8_lib, sym), sym
    import json

    kernels = json.loads((path.parent / "kernel_resources.json").read_text())
    names = [k["kernel"] for k in kernels]
    assert not any("fa_fwd_int8" in n or "int8_scores" in n for n in names), names
    assert any("fa_fwd_f16_pp" in n for n in names)
