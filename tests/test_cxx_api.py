"""The C++ launch API (include/rdnattention.hpp; the reference's
src/rdna/fa2_forward_f16.hpp:12-44 and fa2_forward_int8qk.hpp:10-46), called
from a C++ caller (tests/cxx/cxx_api_caller.cpp) that fills rdna::ForwardParams
and rdna::ForwardParamsInt8QK field by field, as the reference's gates do
(tests/hip_forward_gate.hip:196-228, tests/hip_forward_int8qk_gate.hip:196-232).

CPU: the caller links and loads against the in-tree library; invalid
parameters return -1 with the reason in rdna::lastError() /
rdna::lastErrorInt8QK() (no prefix; the C ABI adds "Attention (...) failed: ").
GPU: rdna::forwardF16 and rdna::forwardInt8QK give results bit-identical to the
C ABI on the same inputs, and the FP16 result is within the parity bar of the
CPU oracle, so the struct layout and field meaning match the C ABI's.
"""
import ctypes
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
CALLER = ROOT / "tests" / "cxx" / "libcxx_api_caller.so"

_VP, _I64P, _U32P = ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_uint32)
_U32, _I32, _F32 = ctypes.c_uint32, ctypes.c_int32, ctypes.c_float


@pytest.fixture(scope="module")
def cxx():
    if not CALLER.exists():
        pytest.fail(f"{CALLER} is not built (run __graft_entry__.build())")
    import rdnattention

    rdnattention._lib_handle()  # the same librdnattention.so the caller links
    c = ctypes.CDLL(str(CALLER))
    c.cxx_forward_f16.argtypes = [_VP] * 6 + [_I64P, _U32P, _F32, _U32, _U32, _I32, _VP, ctypes.c_char_p, _I32]
    c.cxx_forward_f16.restype = _I32
    c.cxx_forward_int8qk.argtypes = [_VP] * 4 + [_I64P, _U32P] + [_F32] * 4 + [_VP, _VP, _U32, _I32, _VP,
                                                                              ctypes.c_char_p, _I32]
    c.cxx_forward_int8qk.restype = _I32
    c.cxx_has_device.restype = _I32
    return c


def _arrays(strides, dims):
    s = (ctypes.c_int64 * 12)(*[int(x) for x in strides])
    d = (ctypes.c_uint32 * 6)(*[int(x) for x in dims])
    return s, d


def _f16(c, q, k, v, o, strides, dims, scale=0.125, causal=0, rope=0, window=-1, cos=None, sin=None, stream=None):
    s, d = _arrays(strides, dims)
    err = ctypes.create_string_buffer(512)
    rc = c.cxx_forward_f16(q, k, v, o, cos, sin, s, d, scale, causal, rope, window, stream, err, 512)
    return rc, err.value.decode()


def _i8(c, q, k, v, o, strides, dims, qsv=None, ksv=None, q_scale=1.0, k_scale=1.0, causal=0, window=-1,
        stream=None):
    s, d = _arrays(strides, dims)
    err = ctypes.create_string_buffer(512)
    rc = c.cxx_forward_int8qk(q, k, v, o, s, d, dims[5] ** -0.5, q_scale, k_scale, 1.0, qsv, ksv, causal, window,
                              stream, err, 512)
    return rc, err.value.decode()


def _host_ptr():
    a = np.zeros(4096 + 16, dtype=np.uint8)
    return a, a.ctypes.data + (-a.ctypes.data) % 16


@pytest.mark.parametrize("dims,msg", [
    ((1, 8, 8, 8, 8, 48), "unsupported head_dim"),
    ((1, 8, 3, 8, 8, 64), "numHeads must be a positive multiple of numKvHeads"),
    ((1, 8, 8, 0, 8, 64), "empty launch grid"),
])
def test_cxx_forward_f16_errors(cxx, dims, msg):
    hold, p = _host_ptr()
    strides = (8 * 8 * 64, 8 * 64, 64) * 4
    rc, err = _f16(cxx, p, p, p, p, strides, dims)
    assert rc == -1
    assert msg in err and not err.startswith("Attention")


def test_cxx_forward_f16_rope_without_tables(cxx):
    hold, p = _host_ptr()
    rc, err = _f16(cxx, p, p, p, p, (8 * 8 * 64, 8 * 64, 64) * 4, (1, 8, 8, 8, 8, 64), rope=1)
    assert rc == -1 and "rot_cos/rot_sin is null" in err


@pytest.mark.parametrize("dims,msg", [
    ((1, 8, 8, 8, 8, 96), "unsupported head_dim (only 64 and 128"),
    ((1, 8, 0, 8, 8, 64), "numHeads must be a positive multiple of numKvHeads"),
])
def test_cxx_forward_int8_errors(cxx, dims, msg):
    hold, p = _host_ptr()
    rc, err = _i8(cxx, p, p, p, p, (8 * 8 * 64, 8 * 64, 64) * 4, dims)
    assert rc == -1
    assert msg in err and not err.startswith("Attention")


def test_cxx_has_device_without_gpu(cxx):
    import torch

    if torch.cuda.is_available():
        pytest.skip("GPU host")
    assert cxx.cxx_has_device() == 0


# --------------------------------------------------------------------------- #
# GPU: bit-identical to the C ABI
# --------------------------------------------------------------------------- #
F16_CASES = [
    # name, B, Hq, Hkv, Sq, Sk, D, causal, window, rope
    ("gqa_causal_rope_d128", 2, 8, 2, 384, 384, 128, 1, -1, True),
    ("window_d64", 1, 4, 4, 300, 300, 64, 0, 64, False),
    ("decode_splitk_d128", 2, 8, 2, 1, 2048, 128, 1, -1, False),
    ("wide_d256_rope", 1, 2, 1, 200, 200, 256, 1, -1, True),
    ("d512_window", 1, 2, 2, 160, 160, 512, 0, 96, False),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", F16_CASES, ids=[c[0] for c in F16_CASES])
def test_cxx_forward_f16_matches_c_abi(gpu, cxx, case):
    import torch

    from tests.gpu_util import assert_f16_parity, forward_raw, gate_rope_tables, log, reference_f16, seeded_inputs

    name, b, hq, hkv, sq, sk, d, causal, window, rope = case
    log(f"cxx f16 {name}")
    q, k, v = seeded_inputs(11, b, hq, hkv, sq, sk, d)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    cos = sin = None
    if rope:
        c_np, s_np = gate_rope_tables(max(sq, sk), d)
        cos, sin = torch.from_numpy(c_np).cuda(), torch.from_numpy(s_np).cuda()
    o_abi = torch.full_like(qd, float("nan"))
    o_cxx = torch.full_like(qd, float("nan"))
    assert forward_raw(qd, kd, vd, o_abi, causal=bool(causal), window=window, cos=cos, sin=sin) == 0
    strides = (*qd.stride()[:3], *kd.stride()[:3], *vd.stride()[:3], *o_cxx.stride()[:3])
    rc, err = _f16(cxx, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o_cxx.data_ptr(), strides,
                   (b, hq, hkv, sq, sk, d), scale=d ** -0.5, causal=causal, rope=1 if rope else 0, window=window,
                   cos=cos.data_ptr() if rope else None, sin=sin.data_ptr() if rope else None,
                   stream=torch.cuda.current_stream().cuda_stream)
    assert rc == 0, err
    torch.cuda.synchronize()
    assert torch.equal(o_cxx.view(torch.int16), o_abi.view(torch.int16)), name
    ref = reference_f16(q, k, v, bool(causal), window,
                        cos=c_np if rope else None, sin=s_np if rope else None)
    assert_f16_parity(o_cxx.float().cpu().numpy(), ref, name)


@pytest.mark.gpu
@pytest.mark.parametrize("per_token", [False, True], ids=["per_tensor", "per_token"])
def test_cxx_forward_int8_matches_c_abi(gpu, cxx, per_token):
    import torch

    from tests.gpu_util import log
    from tests.test_gpu_int8 import forward_i8

    log(f"cxx int8 per_token={per_token}")
    b, hq, hkv, sq, sk, d = 1, 8, 2, 300, 300, 128
    g = torch.Generator().manual_seed(5)
    qi = torch.randint(-127, 128, (b, hq, sq, d), generator=g, dtype=torch.int8).cuda()
    ki = torch.randint(-127, 128, (b, hkv, sk, d), generator=g, dtype=torch.int8).cuda()
    vi = torch.randint(-127, 128, (b, hkv, sk, d), generator=g, dtype=torch.int8).cuda()
    if per_token:
        qs = (torch.rand(b, hq, sq, generator=g) * 0.02 + 0.001).cuda()
        ks = (torch.rand(b, hkv, sk, generator=g) * 0.02 + 0.001).cuda()
    else:
        qs, ks = 0.004, 0.006
    o_abi = torch.full((b, hq, sq, d), float("nan"), dtype=torch.float16, device="cuda")
    o_cxx = torch.full_like(o_abi, float("nan"))
    assert forward_i8(qi, ki, vi, o_abi, qs, ks, 1.0, True, -1) == 0
    strides = (*qi.stride()[:3], *ki.stride()[:3], *vi.stride()[:3], *o_cxx.stride()[:3])
    rc, err = _i8(cxx, qi.data_ptr(), ki.data_ptr(), vi.data_ptr(), o_cxx.data_ptr(), strides,
                  (b, hq, hkv, sq, sk, d), qsv=qs.data_ptr() if per_token else None,
                  ksv=ks.data_ptr() if per_token else None, q_scale=1.0 if per_token else qs,
                  k_scale=1.0 if per_token else ks, causal=1,
                  stream=torch.cuda.current_stream().cuda_stream)
    assert rc == 0, err
    torch.cuda.synchronize()
    assert torch.isfinite(o_cxx.float()).all()
    assert torch.equal(o_cxx.view(torch.int16), o_abi.view(torch.int16))
