"""Per-token V scale (rdna_attention_forward_int8qk_vtoken; an extension: the
reference lists a per-token V scale as missing, FEATURES.md:191, :201-202).

* Exact rows: per-token scales in {1, 2, 4} on V values in [-31, 31] dequantise
  to exact integers, so the kernel must give what the plain INT8 kernel gives
  on the pre-multiplied V: the same scores, maxima and quantised P.  The P V
  sums differ only by this kernel's rounding of each pq * 2^(m - m_ref) to
  fp16 (relative 2^-11 per product, <= 2^-11 * max|v| on the output; the
  plain kernel sums each block in exact int32), so they must agree to 1e-3
  of the V range here, while a misindexed per-token scale (1 vs 4) would be
  off by a sizeable fraction of it.
* Real scales: within 1e-2 max-abs of the oracle's kernel-exact emulation
  (oracle.attention_int8(..., v_token=...)).
* End to end: flash_attn_int8qk_quantized(v_per_token=True) against the
  emulation on the same GPU-quantised tensors, and against fp attention.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import I8_MAX_ABS, errors, log

# name, B, Hq, Hkv, Sq, Sk, D, causal, window, per-token Q/K, strided V
CASES = [
    ("d128_gqa_causal", 2, 8, 2, 300, 300, 128, True, -1, True, False),
    ("d64_window", 1, 4, 4, 256, 256, 64, False, 64, False, False),
    ("d128_kv_longer", 1, 4, 1, 64, 500, 128, True, -1, True, False),
    ("d64_strided_v", 2, 4, 2, 200, 200, 64, True, -1, True, True),
    ("d128_decode", 2, 8, 2, 1, 1000, 128, True, -1, True, False),
]


def _device_v(v_np, strided):
    v = torch.from_numpy(v_np).cuda()
    if not strided:
        return v
    b, h, s, d = v.shape
    big = torch.zeros((b, s, h + 1, d + 32), dtype=torch.int8, device="cuda")
    view = big[:, :, 1:, 16:16 + d].permute(0, 2, 1, 3)
    view.copy_(v)
    return view


def _scales(case, rng):
    name, b, hq, hkv, sq, sk, d, causal, window, ptok, strided = case
    if ptok:
        qs = rng.uniform(0.002, 0.01, (b, hq, sq)).astype(np.float32)
        ks = rng.uniform(0.002, 0.01, (b, hkv, sk)).astype(np.float32)
        return qs, ks
    return 0.004, 0.006


def _run(qi, ki, vi, qs, ks, causal, window, v_token=None):
    import rdnattention as ra

    out = torch.full(qi.shape, float("nan"), dtype=torch.float16, device="cuda")
    dq = torch.from_numpy(qs).cuda() if isinstance(qs, np.ndarray) else qs
    dk = torch.from_numpy(ks).cuda() if isinstance(ks, np.ndarray) else ks
    vt = torch.from_numpy(v_token).cuda() if v_token is not None else None
    ra.attention_int8_forward_into(qi, ki, vi, out, dq, dk, 1.0, is_causal=causal, window_size=window, v_token=vt)
    torch.cuda.synchronize()
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_vtoken_exact_rows_match_plain_kernel(gpu, case):
    name, b, hq, hkv, sq, sk, d, causal, window, ptok, strided = case
    log(f"vtoken exact {name}")
    rng = np.random.default_rng(71)
    qi = rng.integers(-127, 128, (b, hq, sq, d), dtype=np.int8)
    ki = rng.integers(-127, 128, (b, hkv, sk, d), dtype=np.int8)
    w = rng.integers(-31, 32, (b, hkv, sk, d), dtype=np.int8)
    vs = rng.choice(np.array([1.0, 2.0, 4.0], np.float32), size=(b, hkv, sk))
    v_full = (w.astype(np.int32) * vs[..., None].astype(np.int32)).astype(np.int8)
    qs, ks = _scales(case, rng)
    dq, dk = torch.from_numpy(qi).cuda(), torch.from_numpy(ki).cuda()
    a = _run(dq, dk, _device_v(w, strided), qs, ks, causal, window, v_token=vs)
    plain = _run(dq, dk, _device_v(v_full, strided), qs, ks, causal, window)
    assert torch.isfinite(a.float()).all(), name
    got = a.float().cpu().numpy()
    ref = plain.float().cpu().numpy()
    # outputs are in int8 units (v_scale 1): bound by 1e-3 of the V range
    bound = 1e-3 * float(np.abs(v_full).max())
    mx = float(np.abs(got - ref).max())
    log(f"  max |vtoken - plain| = {mx:.3e} (bound {bound:.3e})")
    assert mx <= bound, (name, mx, bound)


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_vtoken_vs_emulation(gpu, case):
    name, b, hq, hkv, sq, sk, d, causal, window, ptok, strided = case
    log(f"vtoken emulation {name}")
    rng = np.random.default_rng(72)
    qi = rng.integers(-127, 128, (b, hq, sq, d), dtype=np.int8)
    ki = rng.integers(-127, 128, (b, hkv, sk, d), dtype=np.int8)
    vi = rng.integers(-127, 128, (b, hkv, sk, d), dtype=np.int8)
    vt = rng.uniform(0.001, 0.03, (b, hkv, sk)).astype(np.float32)
    qs, ks = _scales(case, rng)
    got = _run(torch.from_numpy(qi).cuda(), torch.from_numpy(ki).cuda(), _device_v(vi, strided), qs, ks, causal,
               window, v_token=vt)
    ref = oracle.attention_int8(qi, ki, vi, qs, ks, 1.0, causal=causal, window=window, v_token=vt)
    mx, mean, rel = errors(got.float().cpu().numpy(), ref)
    log(f"  max_abs={mx:.3e} mean_abs={mean:.3e} rel_rms={rel:.3e}")
    assert mx <= I8_MAX_ABS, (name, mx)


@pytest.mark.gpu
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_vtoken_quantized_end_to_end(gpu, causal):
    import rdnattention as ra

    log(f"vtoken end to end causal={causal}")
    g = torch.Generator().manual_seed(73)
    b, hq, hkv, s, d = 1, 8, 2, 400, 128
    q = torch.randn(b, hq, s, d, generator=g).half()
    k = torch.randn(b, hkv, s, d, generator=g).half()
    v = torch.randn(b, hkv, s, d, generator=g).half()
    out = ra.flash_attn_int8qk_quantized(q.cuda(), k.cuda(), v.cuda(), is_causal=causal, v_per_token=True)
    torch.cuda.synchronize()
    qi, ki, qs, ks = ra.quantize_int8_qk_pertoken(q.cuda(), k.cuda())
    vi, vt = ra.quantize_int8_pertoken_v(v.cuda())
    # the GPU quantiser equals the reference's per-token torch formula on the same device tensor
    from tests.test_gpu_quant import torch_pertoken

    ti, ts = torch_pertoken(v.cuda())
    assert torch.equal(vi, ti) and torch.equal(vt, ts)
    ref = oracle.attention_int8(qi.cpu().numpy(), ki.cpu().numpy(), vi.cpu().numpy(), qs.cpu().numpy(),
                                ks.cpu().numpy(), 1.0, causal=causal, v_token=vt.cpu().numpy())
    mx, mean, rel = errors(out.float().cpu().numpy(), ref)
    log(f"  vs emulation max_abs={mx:.3e}")
    assert mx <= I8_MAX_ABS
    fp = oracle.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=causal)
    mx, mean, rel = errors(out.float().cpu().numpy(), fp)
    log(f"  vs fp attention rel_rms={rel:.3e}")
    assert rel < 5e-2


@pytest.mark.gpu
@pytest.mark.parametrize("vs0", [1.0e6, 1.0e-7])
def test_vtoken_extreme_scales(gpu, vs0):
    """A V row whose scale drives v * vs past fp16 (1e6: saturates to
    +-65504) or into fp16 subnormals (1e-7).  Nothing may become NaN or
    infinite -- a masked key times an infinite V would poison every row of its
    tile --, rows that cannot see key 0 (window 2: |i - j| <= 1) must equal the
    run with vs_0 = 1 bit for bit, and causal row 0 (key 0 only) is v'_0,
    within fp16 rounding of the oracle's value."""
    log(f"vtoken extreme scale {vs0:g}")
    rng = np.random.default_rng(74)
    s, d = 24, 64
    qi = rng.integers(-127, 128, (1, 2, s, d), dtype=np.int8)
    ki = rng.integers(-127, 128, (1, 1, s, d), dtype=np.int8)
    vi = rng.integers(-127, 128, (1, 1, s, d), dtype=np.int8)
    vi[0, 0, 0, :8] = 127
    vi[0, 0, 0, 8:16] = -127
    vt = rng.uniform(0.01, 0.03, (1, 1, s)).astype(np.float32)
    vt[0, 0, 0] = vs0
    dq, dk, dv = (torch.from_numpy(x).cuda() for x in (qi, ki, vi))
    got = _run(dq, dk, dv, 0.01, 0.01, True, -1, v_token=vt).float().cpu().numpy()
    assert np.isfinite(got).all()
    ref = oracle.attention_int8(qi, ki, vi, 0.01, 0.01, 1.0, causal=True, v_token=vt)
    np.testing.assert_allclose(got[0, :, 0], ref[0, :, 0], rtol=2e-3, atol=1e-9)
    mx, _, _ = errors(got[:, :, 1:], ref[:, :, 1:])
    assert mx <= I8_MAX_ABS * max(1.0, float(np.abs(ref[:, :, 1:]).max())), mx
    w = _run(dq, dk, dv, 0.01, 0.01, False, 2, v_token=vt)
    vt1 = vt.copy()
    vt1[0, 0, 0] = 1.0
    w1 = _run(dq, dk, dv, 0.01, 0.01, False, 2, v_token=vt1)
    assert torch.isfinite(w.float()).all()
    assert torch.equal(w[:, :, 2:].view(torch.int16), w1[:, :, 2:].view(torch.int16))
