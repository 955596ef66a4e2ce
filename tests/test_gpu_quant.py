"""GPU quantisers and the fused per-channel V rescale.

* rdna_quantize_int8 against the reference wrapper's torch formulas
  (rdnattention/__init__.py:303-343) evaluated by torch on the same device:
  int8 values and fp32 scales bit-identical, for fp16 and fp32 inputs,
  strided views, all-zero rows/columns (scale 1) and exact .5 ties
  (round-half-to-even).
* rdna_attention_forward_int8qk_vchannel against the kernel-exact CPU
  emulation (oracle.attention_int8) times the channel scales, within the
  INT8 bar, and against the unfused composition (kernel, then an fp32
  multiply by v_channel) within fp16 rounding of the output.
* flash_attn_int8qk_quantized (quantisers + fused kernel) against the
  reference's own composition of torch quantisers, flash_attn_int8qk and a
  torch rescale.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import I8_MAX_ABS, errors, log

pytestmark = pytest.mark.gpu


def torch_pertoken(x):
    x = x.float()
    s = x.abs().amax(dim=-1, keepdim=True) / 127.0
    s = torch.where(s == 0, torch.ones_like(s), s)
    return torch.clamp(torch.round(x / s), -127, 127).to(torch.int8), s.squeeze(-1).contiguous()


def torch_perchannel(v):
    v = v.float()
    c = v.abs().amax(dim=-2, keepdim=True) / 127.0
    c = torch.where(c == 0, torch.ones_like(c), c)
    return torch.clamp(torch.round(v / c), -127, 127).to(torch.int8), c.squeeze(-2).contiguous()


def make_x(gpu, shape, dtype, seed, strided):
    g = torch.Generator().manual_seed(seed)
    b, h, s, d = shape
    if strided:
        # a [B, S, 2, H, D] buffer viewed as [B, H, S, D]
        buf = torch.randn(b, s, 2, h, d, generator=g) * 3.0
        x = buf.to(dtype).to(gpu)[:, :, 1].transpose(1, 2)
    else:
        x = (torch.randn(b, h, s, d, generator=g) * 3.0).to(dtype).to(gpu)
    # an all-zero row and an all-zero column (scale 1), and exact ties: row 2
    # has max 63.5 (s = 0.5) and entries 0.25 m, so x / s = m / 2 exactly
    x[0, 0, 0] = 0
    if s > 2:
        x[:, :, :, 1] = 0
        row = torch.arange(d, device=gpu, dtype=torch.float32)
        x[0, 0, 2] = ((row % 9) - 4).to(dtype) * 0.25  # x / s = odd multiples of 0.5 with s = 0.5
        x[0, 0, 2, 0] = 63.5
    return x


SHAPES = [(1, 4, 70, 64), (2, 3, 33, 128), (1, 2, 129, 96), (1, 1, 17, 32), (1, 2, 40, 512), (2, 8, 1000, 128)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("strided", [False, True], ids=["contig", "strided"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{s[2]}x{s[3]}" for s in SHAPES])
def test_pertoken_bit_identical_to_torch(gpu, dtype, strided, shape):
    import rdnattention as ra

    log(f"[quant] pertoken {shape} {dtype} strided={strided}")
    x = make_x(gpu, shape, dtype, 10, strided)
    qi, qs = ra._quantize_gpu(x, per_channel=False)
    ti, ts = torch_pertoken(x)
    torch.cuda.synchronize()
    assert qs.shape == ts.shape and qi.shape == ti.shape
    assert torch.equal(qs, ts)
    assert torch.equal(qi, ti)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("strided", [False, True], ids=["contig", "strided"])
@pytest.mark.parametrize("shape", SHAPES + [(1, 2, 5000, 128), (2, 1, 1, 64)],
                         ids=[f"{s[2]}x{s[3]}" for s in SHAPES + [(1, 2, 5000, 128), (2, 1, 1, 64)]])
def test_perchannel_bit_identical_to_torch(gpu, dtype, strided, shape):
    import rdnattention as ra

    log(f"[quant] perchannel {shape} {dtype} strided={strided}")
    x = make_x(gpu, shape, dtype, 11, strided)
    qi, qc = ra._quantize_gpu(x, per_channel=True)
    ti, tc = torch_perchannel(x)
    torch.cuda.synchronize()
    assert qc.shape == tc.shape and qi.shape == ti.shape
    assert torch.equal(qc, tc)
    assert torch.equal(qi, ti)


def test_public_quantisers_use_the_kernels(gpu):
    """quantize_int8_qk_pertoken / quantize_int8_perchannel_v on HIP tensors
    give the reference formulas' results."""
    import rdnattention as ra

    g = torch.Generator().manual_seed(12)
    q = torch.randn(2, 8, 100, 128, generator=g).half().to(gpu)
    k = torch.randn(2, 2, 100, 128, generator=g).half().to(gpu)
    v = torch.randn(2, 2, 100, 128, generator=g).half().to(gpu)
    qi, ki, qs, ks = ra.quantize_int8_qk_pertoken(q, k)
    for a, b in zip((qi, qs), torch_pertoken(q)):
        assert torch.equal(a, b)
    for a, b in zip((ki, ks), torch_pertoken(k)):
        assert torch.equal(a, b)
    _, _, vi, _, _, vs, vc = ra.quantize_int8_perchannel_v(q, k, v)
    ti, tc = torch_perchannel(v)
    assert vs == 1.0 and torch.equal(vi, ti) and torch.equal(vc, tc)


# b, hq, hkv, s, d, causal, window
VCH_CASES = [(1, 4, 4, 200, 64, False, -1), (1, 8, 2, 300, 128, True, -1), (2, 4, 1, 150, 128, False, 64),
             (1, 8, 8, 1, 64, True, -1)]


@pytest.mark.parametrize("case", VCH_CASES, ids=[f"b{c[0]}h{c[1]}kv{c[2]}s{c[3]}d{c[4]}" for c in VCH_CASES])
def test_vchannel_kernel(gpu, case):
    import rdnattention as ra

    b, hq, hkv, s, d, causal, window = case
    log(f"[quant] vchannel {case}")
    g = torch.Generator().manual_seed(13)
    q = torch.randn(b, hq, s, d, generator=g)
    k = torch.randn(b, hkv, s, d, generator=g)
    v = torch.randn(b, hkv, s, d, generator=g) * torch.linspace(0.2, 3.0, d)  # channels of different range
    qi, qs = oracle.quant_pertoken(q.numpy())
    ki, ks = oracle.quant_pertoken(k.numpy())
    vi, vc = oracle.quant_perchannel(v.numpy())
    emu = oracle.attention_int8(qi, ki, vi, qs, ks, 1.0, causal=causal, window=window)
    emu = emu * np.repeat(vc, hq // hkv, axis=1)[:, :, None, :]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    out = torch.empty(b, hq, s, d, dtype=torch.float16, device=gpu)
    plain = torch.empty_like(out)
    ra.attention_int8_forward_into(t(qi), t(ki), t(vi), out, t(qs), t(ks), 1.0, is_causal=causal,
                                   window_size=window, v_channel=t(vc))
    ra.attention_int8_forward_into(t(qi), t(ki), t(vi), plain, t(qs), t(ks), 1.0, is_causal=causal,
                                   window_size=window)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    mx, mean, _ = errors(o, emu)
    log(f"[quant]   vs emulation max={mx:.2e} mean={mean:.2e}")
    assert mx <= I8_MAX_ABS
    composed = plain.float().cpu().numpy() * np.repeat(vc, hq // hkv, axis=1)[:, :, None, :]
    assert np.allclose(o, composed, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("hkv", [8, 2], ids=["mha", "gqa4"])
def test_quantized_end_to_end_matches_reference_composition(gpu, hkv):
    """flash_attn_int8qk_quantized against the reference's composition
    (rdnattention/__init__.py:346-357): torch quantisers, flash_attn_int8qk
    with v_scale = 1, then out.float() * v_channel -> fp16."""
    import rdnattention as ra

    log(f"[quant] end to end hkv={hkv}")
    g = torch.Generator().manual_seed(14)
    b, hq, s, d = 2, 8, 257, 128
    q = torch.randn(b, hq, s, d, generator=g).half().to(gpu)
    k = torch.randn(b, hkv, s, d, generator=g).half().to(gpu)
    v = torch.randn(b, hkv, s, d, generator=g).half().to(gpu)
    out = ra.flash_attn_int8qk_quantized(q, k, v, is_causal=True)
    qi, qs = torch_pertoken(q)
    ki, ks = torch_pertoken(k)
    vi, vc = torch_perchannel(v)
    ref = ra.flash_attn_int8qk(qi, ki, vi, qs, ks, 1.0, is_causal=True)
    ref = (ref.float() * vc.repeat_interleave(hq // hkv, dim=1).unsqueeze(-2)).half()
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and out.shape == q.shape
    diff = (out.float() - ref.float()).abs()
    log(f"[quant]   vs composition max={diff.max().item():.2e}")
    assert torch.allclose(out.float(), ref.float(), rtol=2e-3, atol=2e-3)


# INT8 with RoPE (an extension: the reference has no INT8 RoPE). The per-token
# quantiser rotates each row with the FP16 path's arithmetic before scaling.
# The oracle rotates in numpy (each product rounded); the kernel may contract a
# product into an FMA, so a rotated value can differ in its last fp16 bit:
# int8 values may then differ by one and scales by an fp16 ulp, rarely.
ROPE_SHAPES = [(1, 4, 70, 64), (2, 3, 33, 128), (1, 2, 300, 256), (1, 2, 40, 512)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("shape", ROPE_SHAPES, ids=[f"{s[2]}x{s[3]}" for s in ROPE_SHAPES])
def test_pertoken_rope_quantiser(gpu, dtype, shape):
    import rdnattention as ra

    log(f"[quant] pertoken rope {shape} {dtype}")
    b, h, s, d = shape
    g = torch.Generator().manual_seed(15)
    x = (torch.randn(b, h, s, d, generator=g) * 3.0).to(dtype)
    cos, sin = oracle.rope_tables(s + 5, d)
    qi, qs = ra._quantize_gpu(x.to(gpu), per_channel=False, rot_cos=torch.from_numpy(cos).to(gpu),
                              rot_sin=torch.from_numpy(sin).to(gpu))
    rot = torch.from_numpy(oracle.rope(x.float().numpy(), cos, sin, round_f16=dtype == torch.float16))
    ti, ts = torch_pertoken(rot.to(dtype).to(gpu))
    torch.cuda.synchronize()
    assert torch.allclose(qs, ts, rtol=2e-3, atol=0)
    di = (qi.int() - ti.int()).abs()
    assert di.max().item() <= 1
    assert (di > 0).float().mean().item() < 2e-3
    # the same rows unrotated are quantised as without tables
    ui, us = ra._quantize_gpu(x.to(gpu), per_channel=False)
    pi, ps = torch_pertoken(x.to(gpu))
    assert torch.equal(ui, pi) and torch.equal(us, ps)


def test_rope_quantiser_rejects_per_channel(gpu):
    import rdnattention as ra

    x = torch.randn(1, 2, 16, 64, device=gpu)
    cos, sin = oracle.rope_tables(16, 64)
    with pytest.raises(ValueError, match="per-token"):
        ra._quantize_gpu(x, per_channel=True, rot_cos=torch.from_numpy(cos).to(gpu),
                         rot_sin=torch.from_numpy(sin).to(gpu))


@pytest.mark.parametrize("causal,hkv", [(True, 2), (False, 8)], ids=["causal_gqa4", "dense_mha"])
def test_quantized_rope_end_to_end(gpu, oracle_lib, causal, hkv):
    """flash_attn_int8qk_quantized with RoPE against the kernel-exact INT8
    emulation of the oracle-rotated, oracle-quantised inputs (INT8 bar, at the
    channel scales)."""
    import rdnattention as ra

    log(f"[quant] rope end to end causal={causal} hkv={hkv}")
    g = torch.Generator().manual_seed(16)
    b, hq, s, d = 2, 8, 300, 128
    q = torch.randn(b, hq, s, d, generator=g).half()
    k = torch.randn(b, hkv, s, d, generator=g).half()
    v = torch.randn(b, hkv, s, d, generator=g).half()
    cos, sin = oracle.rope_tables(s, d)
    out = ra.flash_attn_int8qk_quantized(q.to(gpu), k.to(gpu), v.to(gpu), is_causal=causal,
                                         rot_cos=torch.from_numpy(cos).to(gpu), rot_sin=torch.from_numpy(sin).to(gpu))
    torch.cuda.synchronize()
    qr = oracle.rope(q.float().numpy(), cos, sin, round_f16=True)
    kr = oracle.rope(k.float().numpy(), cos, sin, round_f16=True)
    qi, qsv = oracle.quant_pertoken(qr)
    ki, ksv = oracle.quant_pertoken(kr)
    vi, vc = oracle.quant_perchannel(v.float().numpy())
    emu = oracle.attention_int8(qi, ki, vi, qsv, ksv, 1.0, causal=causal)
    vscale = np.repeat(vc, hq // hkv, axis=1)[:, :, None, :]
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    mx, mean, _ = errors(got, emu * vscale)
    log(f"[quant]   vs emulation max={mx:.2e} mean={mean:.2e}")
    assert mx <= I8_MAX_ABS
