"""The reference's own kernels, compiled for gfx950 from its sources
(oracle/_ref/librdnattention_ref.so, built by ``make -C oracle ref`` from
src/c_api.cpp, src/rdna/fa2_forward_f16.hip and
src/rdna/fa2_forward_int8qk.hip), run on the same inputs as this library.

Two checks per case:
  * reference library vs the CPU oracle: pins the oracle's restatement of the
    reference algorithm against the reference code itself (same bars as the
    HIP path, so an oracle that drifted from the reference would show here);
  * this library vs the reference library: the drop-in claim, output for
    output, through the same C ABI (src/c_api.hpp:16-87).

Running the reference kernels on wave64 hardware is sound: their cross-lane
reductions use DPP quad_perm / row_half_mirror / row_mirror, which act within
16-lane rows on every GCN/CDNA wave size (fa2_forward_f16.hip:28-57); their
blocks are 16x16 threads; every global load and store is guarded by seq_len /
key_seq_len / head validity (fa2_forward_f16.hip:230-295, :690-740, :820-875;
fa2_forward_int8qk.hip:200-220, :450-490).

The reference library is loaded with RTLD_DEEPBIND so that its C entry points
call its own C++ functions (rdna::forwardF16 and friends share their names with
this library's C++ API).

SKIPPED: the first call into the reference library on an MI355X ended the
process with a host segmentation fault inside rdna_attention_forward (before
any output was compared).  Reading the reference's host path, its kernel
resources (no scratch, LDS <= 64 KiB, <= 256 VGPRs) and the dynamic-linker
bindings of both libraries (every HIP symbol binds to the one runtime torch
loaded) has not shown a cause, so these tests stay off the GPU until one is
shown.
"""
import ctypes
import os
import zlib
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import (F16_MAX_ABS, F16_MEAN_ABS, I8_MAX_ABS, errors, forward_raw, gate_rope_tables,
                            lib, log, reference_f16, seeded_inputs, stream_ptr)

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skip(reason="the reference library's first call segfaulted on the host on MI355X; cause not yet "
                            "shown, so it is not run again"),
]

REF_LIB = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "librdnattention_ref.so"
GOLDEN = Path(__file__).resolve().parent / "golden"

_VP, _I64, _U32, _I32, _F32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint32, ctypes.c_int32, ctypes.c_float


@pytest.fixture(scope="module")
def ref():
    if not REF_LIB.exists():
        pytest.skip(f"{REF_LIB} not built (make -C oracle ref needs the reference sources)")
    h = ctypes.CDLL(str(REF_LIB), mode=os.RTLD_LOCAL | os.RTLD_DEEPBIND)
    h.rdna_get_error.argtypes, h.rdna_get_error.restype = [], ctypes.c_char_p
    h.rdna_attention_forward.argtypes = [_VP] * 6 + [_I64] * 12 + [_U32] * 6 + [_F32, _I32, _I32, _I32, _VP]
    h.rdna_attention_forward.restype = _I32
    h.rdna_attention_forward_int8qk.argtypes = ([_VP] * 4 + [_I64] * 12 + [_U32] * 6 + [_F32] * 4
                                               + [_VP, _VP, _I32, _I32, _VP])
    h.rdna_attention_forward_int8qk.restype = _I32
    return h


def ref_f16(h, q, k, v, out, causal, window, cos=None, sin=None):
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    qs, ks, vs, os_ = q.stride(), k.stride(), v.stride(), out.stride()
    rc = h.rdna_attention_forward(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
        cos.data_ptr() if cos is not None else None, sin.data_ptr() if sin is not None else None,
        qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os_[0], os_[1], os_[2],
        b, hq, hkv, sq, sk, d, d ** -0.5, 1 if causal else 0, 1 if cos is not None else 0, int(window), stream_ptr())
    assert rc == 0, h.rdna_get_error()


def i8_call(fn, qi, ki, vi, out, q_scale, k_scale, v_scale, causal, window):
    b, hq, sq, d = qi.shape
    hkv, sk = ki.shape[1], ki.shape[2]
    per_token = isinstance(q_scale, torch.Tensor)
    qs, ks, vs, os_ = qi.stride(), ki.stride(), vi.stride(), out.stride()
    return fn(qi.data_ptr(), ki.data_ptr(), vi.data_ptr(), out.data_ptr(),
              qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os_[0], os_[1], os_[2],
              b, hq, hkv, sq, sk, d, d ** -0.5,
              1.0 if per_token else float(q_scale), 1.0 if per_token else float(k_scale), float(v_scale),
              q_scale.data_ptr() if per_token else None, k_scale.data_ptr() if per_token else None,
              1 if causal else 0, int(window), stream_ptr())


def _check_f16(name, ours, theirs, exact):
    m_ro, a_ro, _ = errors(theirs, exact)
    m_oo, a_oo, _ = errors(ours, exact)
    m_or, a_or, _ = errors(ours, theirs)
    log(f"[ref-lib] {name}: ref-vs-oracle max={m_ro:.2e} mean={a_ro:.2e} | ours-vs-oracle max={m_oo:.2e} "
        f"mean={a_oo:.2e} | ours-vs-ref max={m_or:.2e} mean={a_or:.2e}")
    assert m_ro <= F16_MAX_ABS and a_ro <= F16_MEAN_ABS, f"{name}: reference library vs oracle"
    assert m_oo <= F16_MAX_ABS and a_oo <= F16_MEAN_ABS, f"{name}: this library vs oracle"
    # both sit within the bar of the exact result, so within twice it of each other
    assert m_or <= 2 * F16_MAX_ABS and a_or <= 2 * F16_MEAN_ABS, f"{name}: this library vs reference library"


F16_GOLDEN = sorted(GOLDEN.glob("f16_*.npz"))


@pytest.mark.parametrize("path", F16_GOLDEN, ids=[p.stem for p in F16_GOLDEN])
def test_f16_golden_against_reference_library(gpu, ref, path):
    with np.load(path, allow_pickle=False) as z:
        fx = {k: z[k] for k in z.files}
    b, hq, hkv, sq, sk, d, causal, window, rope = (int(x) for x in fx["params"])
    q, k, v = (torch.from_numpy(fx[n]).to(gpu) for n in ("q", "k", "v"))
    cos = torch.from_numpy(fx["cos"]).to(gpu) if rope else None
    sin = torch.from_numpy(fx["sin"]).to(gpu) if rope else None
    log(f"[ref-lib] golden {path.stem}")
    theirs = torch.empty_like(q)
    ours = torch.empty_like(q)
    ref_f16(ref, q, k, v, theirs, bool(causal), window, cos, sin)
    assert forward_raw(q, k, v, ours, bool(causal), window, cos, sin) == 0
    torch.cuda.synchronize()
    _check_f16(path.stem, ours.float().cpu().numpy(), theirs.float().cpu().numpy(), fx["out"])


# name, b, hq, hkv, sq, sk, d, causal, window, rope
F16_CASES = [
    ("gqa_causal_rope_d128", 1, 8, 2, 1024, 1024, 128, True, -1, True),
    ("mha_dense_tail_d64", 2, 4, 4, 700, 700, 64, False, -1, False),
    ("window_rope_d256", 1, 4, 2, 512, 512, 256, False, 128, True),
    ("causal_d512", 1, 2, 2, 256, 256, 512, True, -1, False),
    ("cross_causal_d96", 1, 4, 4, 100, 333, 96, True, -1, False),
    ("decode_gqa_d128", 4, 32, 8, 1, 4096, 128, True, -1, False),
    ("decode4_gqa_d128", 2, 16, 4, 4, 2048, 128, True, -1, False),
    ("causal_window_gqa_d160", 1, 8, 4, 600, 600, 160, True, 200, False),
]


@pytest.mark.parametrize("case", F16_CASES, ids=[c[0] for c in F16_CASES])
def test_f16_against_reference_library(gpu, ref, case):
    name, b, hq, hkv, sq, sk, d, causal, window, rope = case
    log(f"[ref-lib] {case}")
    q, k, v = seeded_inputs(zlib.crc32(name.encode()) & 0xFFFF, b, hq, hkv, sq, sk, d)
    cos = sin = None
    if rope:
        c, s = gate_rope_tables(max(sq, sk), d)
        cos, sin = torch.from_numpy(c), torch.from_numpy(s)
    exact = reference_f16(q, k, v, causal, window, cos.numpy() if rope else None, sin.numpy() if rope else None)
    q, k, v = q.to(gpu), k.to(gpu), v.to(gpu)
    if rope:
        cos, sin = cos.to(gpu), sin.to(gpu)
    theirs = torch.empty_like(q)
    ours = torch.empty_like(q)
    ref_f16(ref, q, k, v, theirs, causal, window, cos, sin)
    assert forward_raw(q, k, v, ours, causal, window, cos, sin) == 0
    torch.cuda.synchronize()
    _check_f16(name, ours.float().cpu().numpy(), theirs.float().cpu().numpy(), exact)


# name, b, hq, hkv, sq, sk, d, causal, window, per_token
I8_CASES = [
    ("pertoken_causal_gqa_d128", 1, 8, 2, 1024, 1024, 128, True, -1, True),
    ("pertensor_dense_tail_d64", 2, 4, 4, 500, 500, 64, False, -1, False),
    ("pertoken_window_d64", 1, 4, 4, 384, 384, 64, False, 96, True),
    ("pertensor_decode_gqa_d128", 2, 16, 4, 1, 1500, 128, True, -1, False),
]


@pytest.mark.parametrize("case", I8_CASES, ids=[c[0] for c in I8_CASES])
def test_int8_against_reference_library(gpu, ref, case):
    name, b, hq, hkv, sq, sk, d, causal, window, per_token = case
    log(f"[ref-lib] {case}")
    q, k, v = seeded_inputs(zlib.crc32(name.encode()) & 0xFFFF, b, hq, hkv, sq, sk, d)
    qf, kf, vf = q.float().numpy(), k.float().numpy(), v.float().numpy()
    if per_token:
        qi, qsc = oracle.quant_pertoken(qf)
        ki, ksc = oracle.quant_pertoken(kf)
    else:
        qi, qsc = oracle.quant_pertensor(qf)
        ki, ksc = oracle.quant_pertensor(kf)
    vi, vsc = oracle.quant_pertensor(vf)
    exact = oracle.attention_int8(qi, ki, vi, qsc, ksc, vsc, causal=causal, window=window)
    g = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    qt, kt, vt = g(qi), g(ki), g(vi)
    qs_arg = g(qsc) if per_token else qsc
    ks_arg = g(ksc) if per_token else ksc
    theirs = torch.empty(b, hq, sq, d, dtype=torch.float16, device=gpu)
    ours = torch.empty_like(theirs)
    rc = i8_call(ref.rdna_attention_forward_int8qk, qt, kt, vt, theirs, qs_arg, ks_arg, vsc, causal, window)
    assert rc == 0, ref.rdna_get_error()
    assert i8_call(lib().rdna_attention_forward_int8qk, qt, kt, vt, ours, qs_arg, ks_arg, vsc, causal, window) == 0
    torch.cuda.synchronize()
    t = theirs.float().cpu().numpy()
    o = ours.float().cpu().numpy()
    m_ro, a_ro, _ = errors(t, exact)
    m_oo, a_oo, _ = errors(o, exact)
    m_or, a_or, _ = errors(o, t)
    log(f"[ref-lib] {name}: ref-vs-emulation max={m_ro:.2e} mean={a_ro:.2e} | ours-vs-emulation max={m_oo:.2e} "
        f"mean={a_oo:.2e} | ours-vs-ref max={m_or:.2e} mean={a_or:.2e}")
    assert m_ro <= I8_MAX_ABS, f"{name}: reference library vs emulation"
    assert m_oo <= I8_MAX_ABS, f"{name}: this library vs emulation"
    assert m_or <= 2 * I8_MAX_ABS, f"{name}: this library vs reference library"


def _time_ms(fn, reps=3):
    fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / reps


# Full-size workloads, compared library against library (no CPU result at these
# sizes): name, b, hq, hkv, sq, sk, d, causal, rope
FULL_F16 = [
    ("fp16_causal_gqa_rope_b4_h32_kv8_s4096_d128", 4, 32, 8, 4096, 4096, 128, True, True),
    ("fp16_decode_b16_h32_kv8_sq1_sk32768_d128", 16, 32, 8, 1, 32768, 128, True, False),
]


@pytest.mark.parametrize("case", FULL_F16, ids=[c[0] for c in FULL_F16])
def test_f16_full_size_against_reference_library(gpu, ref, case):
    name, b, hq, hkv, sq, sk, d, causal, rope = case
    log(f"[ref-lib] full size {case}")
    g = torch.Generator(device=gpu).manual_seed(zlib.crc32(name.encode()))
    q = torch.randn(b, hq, sq, d, generator=g, device=gpu, dtype=torch.float16)
    k = torch.randn(b, hkv, sk, d, generator=g, device=gpu, dtype=torch.float16)
    v = torch.randn(b, hkv, sk, d, generator=g, device=gpu, dtype=torch.float16)
    cos = sin = None
    if rope:
        c, s = gate_rope_tables(max(sq, sk), d)
        cos, sin = torch.from_numpy(c).to(gpu), torch.from_numpy(s).to(gpu)
    theirs = torch.empty_like(q)
    ours = torch.empty_like(q)
    t_ref = _time_ms(lambda: ref_f16(ref, q, k, v, theirs, causal, -1, cos, sin))
    t_ours = _time_ms(lambda: forward_raw(q, k, v, ours, causal, -1, cos, sin))
    flops = oracle.attn_flops(b, hq, sq, sk, d, causal, -1)
    diff = (ours.float() - theirs.float()).abs()
    mx, mean = diff.max().item(), diff.mean().item()
    log(f"[ref-lib] {name}: reference {t_ref:.3f} ms ({flops / t_ref / 1e9:.1f} TFLOP/s) | this library "
        f"{t_ours:.3f} ms ({flops / t_ours / 1e9:.1f} TFLOP/s) | speedup {t_ref / t_ours:.1f}x | "
        f"ours-vs-ref max={mx:.2e} mean={mean:.2e}")
    assert torch.isfinite(ours).all()
    assert mx <= 2 * F16_MAX_ABS and mean <= 2 * F16_MEAN_ABS


def test_int8_full_size_against_reference_library(gpu, ref):
    name, b, hq, hkv, s, d = "int8_causal_gqa_pertoken_b2_h32_kv8_s8192_d128", 2, 32, 8, 8192, 128
    log(f"[ref-lib] full size {name}")
    import rdnattention

    g = torch.Generator(device=gpu).manual_seed(zlib.crc32(name.encode()))
    q = torch.randn(b, hq, s, d, generator=g, device=gpu, dtype=torch.float16)
    k = torch.randn(b, hkv, s, d, generator=g, device=gpu, dtype=torch.float16)
    v = torch.randn(b, hkv, s, d, generator=g, device=gpu, dtype=torch.float16)
    qi, ki, qsc, ksc = rdnattention.quantize_int8_qk_pertoken(q, k)
    vsc = v.float().abs().max().item() / 127.0
    vi = torch.clamp(torch.round(v.float() / vsc), -127, 127).to(torch.int8)
    del q, k, v
    theirs = torch.empty(b, hq, s, d, dtype=torch.float16, device=gpu)
    ours = torch.empty_like(theirs)

    def run(fn, out):
        assert i8_call(fn, qi, ki, vi, out, qsc, ksc, vsc, True, -1) == 0

    t_ref = _time_ms(lambda: run(ref.rdna_attention_forward_int8qk, theirs))
    t_ours = _time_ms(lambda: run(lib().rdna_attention_forward_int8qk, ours))
    ops = oracle.attn_flops(b, hq, s, s, d, True, -1)
    diff = (ours.float() - theirs.float()).abs()
    mx, mean = diff.max().item(), diff.mean().item()
    log(f"[ref-lib] {name}: reference {t_ref:.3f} ms ({ops / t_ref / 1e9:.1f} TOP/s) | this library "
        f"{t_ours:.3f} ms ({ops / t_ours / 1e9:.1f} TOP/s) | speedup {t_ref / t_ours:.1f}x | "
        f"ours-vs-ref max={mx:.2e} mean={mean:.2e}")
    assert torch.isfinite(ours).all()
    assert mx <= 2 * I8_MAX_ABS
