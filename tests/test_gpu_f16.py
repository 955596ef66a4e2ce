"""FP16 parity on the GPU: librdnattention.so (through the C ABI and the
Python wrapper) against the CPU oracle on the same inputs.

Case lists restate the reference's own suites:
  * GATE_CASES   -- tests/hip_forward_gate.hip:259-316 (50 cases, LCG seed 12345)
  * HEAD_DIM_VARIANTS -- tests/head_dim.py:10-20 (9 variants x 16 head dims, seed 1234)
  * ROPE_CASES   -- tests/rope.py:66-73 (7 cases, seed 7)
Bars: max-abs <= 2e-3, mean-abs <= 2e-4 and the gate's rel_rms < 5e-3.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import (assert_f16_parity, forward_raw, gate_rope_tables, lcg_inputs, log, reference_f16,
                            seeded_inputs)

pytestmark = pytest.mark.gpu

# name, batch, numHeads, numKvHeads, seqLen, keySeqLen, headDim, causal, windowSize, hasRope
GATE_CASES = [
    ("d64_dense_small", 1, 4, 4, 96, 96, 64, False, 0, False),
    ("d64_dense_tail", 2, 4, 4, 200, 200, 64, False, 0, False),
    ("d64_causal", 1, 4, 4, 257, 257, 64, True, 0, False),
    ("d64_gqa_causal", 1, 8, 2, 300, 300, 64, True, 0, False),
    ("d64_gqa_ratio2_exact", 1, 8, 4, 300, 300, 64, True, 0, False),
    ("d64_gqa_ratio8", 1, 16, 2, 300, 300, 64, True, 0, False),
    ("d64_gqa_ratio3_pad", 2, 6, 2, 257, 257, 64, True, 0, False),
    ("d64_gqa_ratio6_even", 1, 12, 2, 300, 300, 64, False, 0, False),
    ("d64_gqa_ratio5_pad", 2, 10, 2, 199, 199, 64, True, 64, True),
    ("d64_gqa_batch4", 4, 8, 2, 96, 96, 64, False, 0, False),
    ("d64_mqa", 2, 8, 1, 199, 199, 64, True, 0, False),
    ("d64_gqa_decode_1tok", 1, 8, 2, 1, 300, 64, False, 0, False),
    ("d64_gqa_decode_few", 2, 16, 4, 4, 300, 64, False, 0, False),
    ("d64_gqa_window", 1, 8, 2, 300, 300, 64, False, 64, False),
    ("d64_gqa_numkv8", 1, 32, 8, 256, 256, 64, True, 0, True),
    ("d64_window", 1, 4, 4, 300, 300, 64, False, 64, False),
    ("d64_causal_window", 1, 4, 4, 300, 300, 64, True, 32, False),
    ("d64_rope_causal", 2, 4, 4, 271, 271, 64, True, 0, True),
    ("d64_kv_longer", 1, 4, 4, 64, 300, 64, False, 0, False),
    ("d128_dense", 1, 4, 4, 130, 130, 128, False, 0, False),
    ("d128_causal", 1, 4, 4, 150, 150, 128, True, 0, False),
    ("d128_rope_gqa_causal", 1, 8, 4, 199, 199, 128, True, 0, True),
    ("d32_dense", 1, 2, 2, 100, 100, 32, False, 0, False),
    ("d96_dense", 1, 2, 2, 100, 100, 96, False, 0, False),
    ("d160_dense", 1, 2, 2, 100, 100, 160, False, 0, False),
    ("d192_dense", 1, 2, 2, 100, 100, 192, False, 0, False),
    ("d224_dense", 1, 2, 2, 100, 100, 224, False, 0, False),
    ("d256_dense", 1, 2, 2, 100, 100, 256, False, 0, False),
    ("d288_dense", 1, 2, 2, 100, 100, 288, False, 0, False),
    ("d320_dense", 1, 2, 2, 100, 100, 320, False, 0, False),
    ("d352_dense", 1, 2, 2, 100, 100, 352, False, 0, False),
    ("d384_dense", 1, 2, 2, 100, 100, 384, False, 0, False),
    ("d416_dense", 1, 2, 2, 100, 100, 416, False, 0, False),
    ("d448_dense", 1, 2, 2, 100, 100, 448, False, 0, False),
    ("d480_dense", 1, 2, 2, 100, 100, 480, False, 0, False),
    ("d512_dense", 1, 2, 2, 100, 100, 512, False, 0, False),
    ("d384_causal", 1, 2, 2, 100, 100, 384, True, 0, False),
    ("d384_gqa_causal", 1, 8, 2, 100, 100, 384, True, 0, False),
    ("d384_window", 1, 2, 2, 100, 100, 384, False, 32, False),
    ("d384_causal_window", 1, 2, 2, 100, 100, 384, True, 32, False),
    ("d384_rope_causal", 1, 2, 2, 100, 100, 384, True, 0, True),
    ("d384_kv_longer", 1, 2, 2, 40, 100, 384, False, 0, False),
    ("d384_decode_1tok", 1, 4, 2, 1, 100, 384, False, 0, False),
    ("d512_causal", 1, 2, 2, 100, 100, 512, True, 0, False),
    ("d512_gqa_rope_causal", 1, 4, 2, 100, 100, 512, True, 0, True),
    ("d512_window", 1, 2, 2, 100, 100, 512, False, 32, False),
    ("d512_kv_longer", 1, 2, 2, 40, 100, 512, False, 0, False),
    ("d256_rope_causal", 1, 2, 2, 100, 100, 256, True, 0, True),
    ("d256_gqa_window", 1, 8, 2, 100, 100, 256, False, 32, False),
    ("d352_causal_aligned", 1, 2, 2, 96, 96, 352, True, 0, False),
]


@pytest.mark.parametrize("case", GATE_CASES, ids=[c[0] for c in GATE_CASES])
def test_gate_cases(gpu, oracle_lib, case):
    name, b, hq, hkv, sq, sk, d, causal, window, rope = case
    log(f"[gate] {name}")
    q, k, v = lcg_inputs(12345, b, hq, hkv, sq, sk, d, mode=0)
    cos = sin = None
    if rope:
        cos, sin = gate_rope_tables(max(sq, sk), d)
    ref = reference_f16(q, k, v, causal, window, cos, sin)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    out = torch.empty_like(qd)
    rc = forward_raw(qd, kd, vd, out, causal, window,
                     torch.from_numpy(cos).to(gpu) if rope else None,
                     torch.from_numpy(sin).to(gpu) if rope else None)
    assert rc == 0
    torch.cuda.synchronize()
    assert_f16_parity(out.float().cpu().numpy(), ref, name)


HEAD_DIM_VARIANTS = [
    ("dense", 1, 300, 300, False, -1),
    ("causal", 1, 300, 300, True, -1),
    ("gqa", 4, 300, 300, False, -1),
    ("gqa_causal", 4, 300, 300, True, -1),
    ("window", 1, 300, 300, False, 64),
    ("causal_window", 1, 300, 300, True, 32),
    ("cross", 1, 200, 300, False, -1),
    ("decode", 1, 1, 300, False, -1),
    ("aligned", 1, 256, 256, True, -1),
]


@pytest.mark.parametrize("d", list(range(32, 513, 32)))
@pytest.mark.parametrize("variant", HEAD_DIM_VARIANTS, ids=[v[0] for v in HEAD_DIM_VARIANTS])
def test_head_dim_python_path(gpu, oracle_lib, d, variant):
    """tests/head_dim.py through rdnattention.flash_attn (8 heads, N(0,1))."""
    import rdnattention

    name, kvdiv, s_len, ks_len, causal, window = variant
    torch.manual_seed(1234)
    h = 8
    kvh = max(1, h // kvdiv)
    q = torch.randn(1, h, s_len, d, dtype=torch.float16)
    k = torch.randn(1, kvh, ks_len, d, dtype=torch.float16)
    v = torch.randn(1, kvh, ks_len, d, dtype=torch.float16)
    out = rdnattention.flash_attn(q.to(gpu), k.to(gpu), v.to(gpu), is_causal=causal, window_size=window)
    torch.cuda.synchronize()
    ref = reference_f16(q, k, v, causal, window)
    assert_f16_parity(out.float().cpu().numpy(), ref, f"d{d}_{name}")


ROPE_CASES = [
    ("MHA d64 rope", 1, 8, 8, 256, 256, 64, False),
    ("MHA d128 rope", 2, 8, 8, 512, 512, 128, False),
    ("causal d64 rope", 1, 8, 8, 256, 256, 64, True),
    ("causal d128 rope", 1, 8, 8, 384, 384, 128, True),
    ("GQA d64 rope", 1, 8, 2, 256, 256, 64, False),
    ("cross-attn d64 rope", 1, 8, 8, 128, 512, 64, False),
    ("tail 300 rope", 1, 8, 8, 300, 300, 64, False),
]


@pytest.mark.parametrize("case", ROPE_CASES, ids=[c[0] for c in ROPE_CASES])
def test_rope_cases(gpu, oracle_lib, case):
    """tests/rope.py:66-96 through rdnattention.flash_attn with in-kernel RoPE."""
    import rdnattention

    name, b, h, kh, s, ks, d, causal = case
    torch.manual_seed(7)
    q = torch.randn(b, h, s, d, dtype=torch.float16)
    k = torch.randn(b, kh, ks, d, dtype=torch.float16)
    v = torch.randn(b, kh, ks, d, dtype=torch.float16)
    cos, sin = oracle.rope_tables(max(s, ks), d)
    out = rdnattention.flash_attn(q.to(gpu), k.to(gpu), v.to(gpu), is_causal=causal,
                                      rot_cos=torch.from_numpy(cos).to(gpu), rot_sin=torch.from_numpy(sin).to(gpu))
    torch.cuda.synchronize()
    ref = reference_f16(q, k, v, causal, -1, cos, sin)
    assert_f16_parity(out.float().cpu().numpy(), ref, name)
    # the reference's own bar against an un-rounded RoPE (tests/rope.py:92-95)
    ref_fp32_rope = oracle.attention(oracle.rope(q.float().numpy(), cos, sin, round_f16=False),
                                     oracle.rope(k.float().numpy(), cos, sin, round_f16=False), v.float().numpy(),
                                     causal=causal)
    got = out.float().cpu().numpy().astype(np.float64)
    rel = np.sqrt(((got - ref_fp32_rope) ** 2).mean() / (ref_fp32_rope ** 2).mean())
    assert rel < 1e-2


def test_quick_start_shape(gpu, oracle_lib):
    """B=1, H=8, S=512, D=64, non-causal, N(0,1) seed 0."""
    q, k, v = seeded_inputs(0, 1, 8, 8, 512, 512, 64)
    out = torch.empty_like(q, device=gpu)
    assert forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out) == 0
    torch.cuda.synchronize()
    assert_f16_parity(out.float().cpu().numpy(), reference_f16(q, k, v, False, -1), "quick_start")


def test_strided_kv_views_bit_identical(gpu, oracle_lib):
    """K/V as head-strided views of one [B,S,2,Hkv,D] buffer: the result is
    bit-identical to contiguous copies and matches the oracle."""
    g = torch.Generator().manual_seed(3)
    b, hq, hkv, sq, sk, d = 2, 8, 2, 37, 333, 128
    buf = torch.randn(b, sk, 2, hkv, d, generator=g).half().to(gpu)
    q = torch.randn(b, hq, sq, d, generator=g).half().to(gpu)
    kv_k = buf[:, :, 0].transpose(1, 2)
    kv_v = buf[:, :, 1].transpose(1, 2)
    assert not kv_k.is_contiguous()
    o1 = torch.empty_like(q)
    o2 = torch.empty_like(q)
    assert forward_raw(q, kv_k, kv_v, o1) == 0
    assert forward_raw(q, kv_k.contiguous(), kv_v.contiguous(), o2) == 0
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    ref = reference_f16(q.cpu(), kv_k.cpu(), kv_v.cpu(), False, -1)
    assert_f16_parity(o1.float().cpu().numpy(), ref, "strided")


def test_strided_output_and_query(gpu, oracle_lib):
    """Q and O as [B,S,H,D]-layout views (seq stride H*D)."""
    g = torch.Generator().manual_seed(4)
    b, h, s, d = 2, 4, 65, 64
    qb = torch.randn(b, s, h, d, generator=g).half().to(gpu)
    kb = torch.randn(b, s, h, d, generator=g).half().to(gpu)
    vb = torch.randn(b, s, h, d, generator=g).half().to(gpu)
    ob = torch.zeros(b, s, h, d, dtype=torch.float16, device=gpu)
    q, k, v, o = (t.transpose(1, 2) for t in (qb, kb, vb, ob))
    assert forward_raw(q, k, v, o, causal=True) == 0
    torch.cuda.synchronize()
    ref = reference_f16(q.cpu(), k.cpu(), v.cpu(), True, -1)
    assert_f16_parity(o.float().cpu().numpy(), ref, "strided_o")


def test_rows_without_keys_are_zero(gpu, oracle_lib):
    """Causal with Sq > Sk: the first Sq - Sk rows see no key and are written as 0."""
    q, k, v = seeded_inputs(5, 1, 2, 2, 100, 40, 64)
    out = torch.full_like(q, 7.0, device=gpu)
    assert forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out, causal=True) == 0
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    assert np.all(o[:, :, :60] == 0.0)
    assert_f16_parity(o, reference_f16(q, k, v, True, -1), "no_keys")


# head dims of every prefill kernel family (all built with -fno-honor-nans:
# an all-masked row must not produce -inf - -inf): 8-wave ping-pong (<= 128),
# key pairs (160-256), head-dimension pairs (288-512); GQA ratio 2
@pytest.mark.parametrize("d", [32, 128, 160, 192, 224, 256, 320, 512])
@pytest.mark.parametrize("mode", ["causal_sq_gt_sk", "window_misses_rows", "causal_window_gqa"])
def test_rows_without_keys_every_kernel(gpu, oracle_lib, d, mode):
    """Rows that see no key are written as 0, and every other row matches the
    oracle: causal with Sq > Sk (the first Sq - Sk rows); a two-sided window
    with Sq > Sk whose band misses the whole key range for the first rows; a
    causal window (GQA) where Sq > Sk leaves rows without keys and the window
    cuts the rest (several key tiles, so masked, mask-free and skipped tiles
    all occur).  The output is pre-filled with 7 so an unwritten row fails."""
    sq, sk, causal, window = {"causal_sq_gt_sk": (300, 100, True, -1),
                              "window_misses_rows": (600, 100, False, 64),
                              "causal_window_gqa": (400, 330, True, 48)}[mode]
    hq, hkv = (4, 2) if mode == "causal_window_gqa" else (2, 2)
    log(f"[f16 empty rows] d{d} {mode} sq{sq} sk{sk}")
    q, k, v = seeded_inputs(31, 1, hq, hkv, sq, sk, d)
    out = torch.full_like(q, 7.0, device=gpu)
    assert forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out, causal, window) == 0
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    ref = reference_f16(q, k, v, causal, window)
    empty = np.all(ref == 0.0, axis=(0, 1, 3))
    n_empty = {"causal_sq_gt_sk": 200, "window_misses_rows": 468, "causal_window_gqa": 70}[mode]
    assert int(empty.sum()) == n_empty and empty[:n_empty].all()
    assert np.all(o[:, :, empty] == 0.0)
    assert_f16_parity(o, ref, f"no_keys d{d} {mode}")


@pytest.mark.parametrize("d", [128, 256, 512])
def test_first_causal_row_exact(gpu, d):
    q, k, v = seeded_inputs(6, 1, 4, 4, 128, 128, d)
    out = torch.empty_like(q, device=gpu)
    assert forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out, causal=True) == 0
    torch.cuda.synchronize()
    assert torch.equal(out[:, :, 0].cpu(), v[:, :, 0])


def test_negative_and_zero_scale(gpu, oracle_lib):
    """`scale` is honoured as passed through the C ABI, including <= 0."""
    q, k, v = seeded_inputs(8, 1, 2, 2, 70, 90, 64)
    for scale in (-0.125, 0.0, 0.3):
        out = torch.empty_like(q, device=gpu)
        assert forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out, causal=True, scale=scale) == 0
        torch.cuda.synchronize()
        ref = oracle.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=True, scale=scale)
        assert_f16_parity(out.float().cpu().numpy(), ref, f"scale={scale}")


def test_empty_key_sequence_outputs_zero(gpu):
    q = torch.randn(1, 2, 10, 64, dtype=torch.float16, device=gpu)
    k = torch.empty(1, 2, 0, 64, dtype=torch.float16, device=gpu)
    out = torch.full_like(q, 3.0)
    assert forward_raw(q, k, k, out) == 0
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0


@pytest.mark.parametrize("d,sq,sk", [(512, 70, 20), (384, 40, 32), (448, 33, 33), (480, 130, 64), (512, 200, 45)])
def test_pair_kernel_few_key_tiles(gpu, oracle_lib, d, sq, sk):
    """The D 384-512 kernel with one or two 32-key tiles (its prologue DMAs
    one or two tile pairs, and the first in-loop DMA issue is skipped), full
    and partial tiles, causal with Sq != Sk."""
    q, k, v = seeded_inputs(17, 1, 4, 2, sq, sk, d)
    out = torch.full_like(q, float("nan"), device=gpu)
    assert forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out, True, -1) == 0
    torch.cuda.synchronize()
    ref = reference_f16(q, k, v, True, -1)
    assert_f16_parity(out.float().cpu().numpy(), ref, f"few_tiles d{d} {sq}x{sk}")


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,sk", [(70, 20), (40, 64), (130, 100), (200, 150)])
@pytest.mark.parametrize("d", [128, 224, 256])
def test_dma_staged_kernels_few_key_tiles(gpu, oracle_lib, d, sq, sk, causal):
    """The kernels whose K/V tiles arrive by DMA from both groups (D = 128:
    the ping-pong kernel; D = 224, 256: the key-pair kernel) with one, two and
    three 64-key tiles, full and partial: group B's prologue and phase-0 K
    DMAs, group A's first V DMA and the skipped in-loop K issues near the
    end; causal with Sq > Sk leaves rows that see no key."""
    q, k, v = seeded_inputs(23, 1, 4, 2, sq, sk, d)
    out = torch.full_like(q, float("nan"), device=gpu)
    assert forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out, causal, -1) == 0
    torch.cuda.synchronize()
    ref = reference_f16(q, k, v, causal, -1)
    assert_f16_parity(out.float().cpu().numpy(), ref, f"dma_few_tiles d{d} {sq}x{sk} causal={causal}")


@pytest.mark.parametrize("d,s,window", [(256, 2048, 1024), (512, 1024, 1024), (416, 640, 256)])
def test_large_head_window_rope_slice(gpu, oracle_lib, d, s, window):
    """The large-head window workloads (two-sided window, RoPE, N(0, 0.5)) at
    a size the oracle finishes quickly; D = 416 runs the head-dimension pair
    kernel with unequal halves (224 + 192 of the head dimension)."""
    q, k, v = seeded_inputs(4, 1, 2, 2, s, s, d, std=0.5)
    cos, sin = oracle.rope_tables(s, d)
    out = torch.empty_like(q, device=gpu)
    assert forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out, False, window, torch.from_numpy(cos).to(gpu),
                       torch.from_numpy(sin).to(gpu)) == 0
    torch.cuda.synchronize()
    ref = reference_f16(q, k, v, False, window, cos, sin)
    assert_f16_parity(out.float().cpu().numpy(), ref, f"d{d}_window{window}")


# d, hq, hkv, sq, sk, causal, window: the D 160-256 and D 384-512 pair
# kernels start each row tile's key-tile walk at the highest band start of its
# block of 32 row tiles (when that tile is in its own band) and wrap around;
# these cover more than one block (row tiles of 128 / G rows), offsets 0 and
# non-zero in one block, a causal window, Sq != Sk, GQA, and a window wider
# than the keys
WALK_CASES = [
    (160, 2, 2, 4500, 4500, False, 700),
    (224, 8, 2, 5000, 5000, True, 1000),
    (256, 3, 3, 3000, 3500, False, 600),
    (192, 4, 4, 2600, 2600, False, 6000),
    (512, 2, 2, 4500, 4500, False, 700),
    (416, 4, 2, 4200, 4400, True, 900),
]


@pytest.mark.parametrize("case", WALK_CASES, ids=lambda c: f"d{c[0]}_h{c[1]}kv{c[2]}_s{c[3]}x{c[4]}_w{c[6]}")
def test_pair_kernel_window_walk(gpu, oracle_lib, case):
    d, hq, hkv, sq, sk, causal, window = case
    q, k, v = seeded_inputs(11, 1, hq, hkv, sq, sk, d, std=0.5)
    out = torch.empty_like(q, device=gpu)
    assert forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out, causal, window) == 0
    torch.cuda.synchronize()
    ref = reference_f16(q, k, v, causal, window)
    assert_f16_parity(out.float().cpu().numpy(), ref, f"walk_d{d}_w{window}")


@pytest.mark.parametrize("d,hq,hkv", [(384, 6, 2), (416, 6, 3), (480, 8, 2), (512, 9, 3), (448, 4, 4)])
def test_wave_pair_split_gqa(gpu, oracle_lib, d, hq, hkv):
    """The head-dimension pair kernel (D > 352) with one head per workgroup
    (odd GQA ratios and MHA), two (ratio 2 mod 4) and four (ratios divisible
    by 4), causal with RoPE, ragged row and key counts, equal and unequal
    halves of the head dimension."""
    log(f"[split] d{d} hq{hq} hkv{hkv}")
    q, k, v = seeded_inputs(15, 2, hq, hkv, 150, 213, d)
    cos, sin = oracle.rope_tables(213, d)
    out = torch.full_like(q, float("nan"), device=gpu)
    assert forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out, True, -1, torch.from_numpy(cos).to(gpu),
                       torch.from_numpy(sin).to(gpu)) == 0
    torch.cuda.synchronize()
    ref = reference_f16(q, k, v, True, -1, cos, sin)
    assert_f16_parity(out.float().cpu().numpy(), ref, f"split d{d} gqa {hq}/{hkv}")


@pytest.mark.parametrize("d", [160, 224, 256, 288, 512])
def test_large_head_strided_kv_bit_identical(gpu, oracle_lib, d):
    """Large-head kernels with K/V sliced from one [B,S,2,Hkv,D] buffer: the
    wave-pair kernel's register staging (160) and two-row DMA staging (224,
    256, where a DMA's second row is one sequence stride past the first) and
    the head-dimension pair kernel (288, 512)."""
    g = torch.Generator().manual_seed(9)
    b, hq, hkv, sq, sk = 1, 4, 2, 70, 133
    buf = torch.randn(b, sk, 2, hkv, d, generator=g).half().to(gpu)
    q = torch.randn(b, hq, sq, d, generator=g).half().to(gpu)
    kv_k = buf[:, :, 0].transpose(1, 2)
    kv_v = buf[:, :, 1].transpose(1, 2)
    o1 = torch.empty_like(q)
    o2 = torch.empty_like(q)
    assert forward_raw(q, kv_k, kv_v, o1, causal=True) == 0
    assert forward_raw(q, kv_k.contiguous(), kv_v.contiguous(), o2, causal=True) == 0
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert_f16_parity(o1.float().cpu().numpy(), reference_f16(q.cpu(), kv_k.cpu(), kv_v.cpu(), True, -1),
                      f"strided_d{d}")


def spike_inputs(seed, b, hq, hkv, s, d, jump, positions):
    """N(0,1) Q/K/V plus a shared direction u: every query carries 4u and the
    keys at `positions` carry delta*u, so their scores exceed the typical row
    max by about `jump` (log2 units) in tiles well after the first."""
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(d, generator=g)
    u = u / u.norm()
    q = torch.randn(b, hq, s, d, generator=g) + 4.0 * u
    k = torch.randn(b, hkv, s, d, generator=g)
    v = torch.randn(b, hkv, s, d, generator=g)
    delta = (jump + 4.0) * d ** 0.5 / (4.0 * 1.4426950408889634)
    for pos in positions:
        k[:, :, pos] = delta * u
    return q.half(), k.half(), v.half()


@pytest.mark.parametrize("d", [64, 128, 256, 384, 512])
@pytest.mark.parametrize("jump", [6.0, 12.0, 20.0, 60.0])
@pytest.mark.parametrize("causal", [False, True])
def test_late_score_spike(gpu, oracle_lib, d, jump, causal):
    """Row maxima that rise far above the running max in later tiles: the
    rescale paths (growth inside the lazy margin, beyond it, and beyond the
    fp16 range of P) must all give the exact softmax.  In the D 288-512
    kernel the spikes at keys 150 and 251 fall in the second half of their
    32-key tiles and the one at 300 in the first, so each half of a wave pair
    raises its reference alone (D 384 with Q pre-scaled, D 512 without)."""
    log(f"[spike] d={d} jump={jump} causal={causal}")
    q, k, v = spike_inputs(11, 1, 4, 2, 320, d, jump, (150, 251, 300))
    out = torch.empty_like(q, device=gpu)
    assert forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out, causal=causal) == 0
    torch.cuda.synchronize()
    ref = reference_f16(q, k, v, causal, -1)
    assert_f16_parity(out.float().cpu().numpy(), ref, f"spike d{d} jump{jump}")


# Row-tile work items well beyond what the device holds at once (at most 512
# workgroups of these kernels on 256 CUs), so every persistent workgroup walks
# several items, with ragged sequence ends and items of unequal size.
# name, b, hq, hkv, s, d, causal, window, rope
PERSISTENT_CASES = [
    ("d128_gqa4_causal_rope", 4, 32, 8, 1100, 128, True, -1, True),     # 32 head groups x 18 row tiles
    ("d96_gqa4_causal_window", 4, 32, 8, 1500, 96, True, 200, False),   # 32 x 24
    ("d64_mha_window", 2, 16, 16, 3000, 64, False, 500, False),         # 32 x 12
    ("d32_gqa2_dense", 4, 16, 8, 2100, 32, False, -1, False),           # 32 x 17
    ("d128_mqa_causal", 1, 16, 1, 2500, 128, True, -1, True),           # 4 x 40
    # the wave-pair kernel (D 160-256), one workgroup per CU
    ("d256_mha_window_rope", 1, 16, 16, 3000, 256, False, 1000, True),  # 16 x 24
    ("d224_gqa2_causal", 2, 16, 8, 2100, 224, True, -1, False),         # 16 x 33
    ("d160_gqa4_window", 1, 16, 4, 2600, 160, True, 700, True),         # 4 x 82
]


@pytest.mark.parametrize("case", PERSISTENT_CASES, ids=[c[0] for c in PERSISTENT_CASES])
def test_persistent_workgroups_cover_every_tile(gpu, oracle_lib, case):
    """Output pre-filled with NaN: a row tile that no workgroup writes fails
    the finiteness check, one written wrongly fails the FP16 bar."""
    name, b, hq, hkv, s, d, causal, window, rope = case
    log(f"[persistent] {name}")
    q, k, v = seeded_inputs(21, b, hq, hkv, s, s, d)
    cos = sin = None
    if rope:
        cos, sin = oracle.rope_tables(s, d)
    out = torch.full_like(q, float("nan"), device=gpu)
    rc = forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out, causal, window,
                     torch.from_numpy(cos).to(gpu) if rope else None,
                     torch.from_numpy(sin).to(gpu) if rope else None, path=1)
    assert rc == 0
    torch.cuda.synchronize()
    assert_f16_parity(out.float().cpu().numpy(), reference_f16(q, k, v, causal, window, cos, sin), name)


def test_scratch_trim_between_calls(gpu, oracle_lib):
    """trim_scratch() returns the pooled RoPE scratch to the device; calls
    before and after it give bit-identical results."""
    import rdnattention

    q, k, v = seeded_inputs(16, 1, 8, 2, 700, 700, 128)
    cos, sin = oracle.rope_tables(700, 128)
    cd, sd = torch.from_numpy(cos).to(gpu), torch.from_numpy(sin).to(gpu)
    a = rdnattention.flash_attn(q.to(gpu), k.to(gpu), v.to(gpu), is_causal=True, rot_cos=cd, rot_sin=sd)
    rdnattention.trim_scratch()
    b = rdnattention.flash_attn(q.to(gpu), k.to(gpu), v.to(gpu), is_causal=True, rot_cos=cd, rot_sin=sd)
    torch.cuda.synchronize()
    rdnattention.trim_scratch()
    assert torch.equal(a, b)
    assert_f16_parity(a.float().cpu().numpy(), reference_f16(q, k, v, True, -1, cos, sin), "trim")


@pytest.mark.gpu
def test_cached_scratch_two_streams_and_growth(gpu, oracle_lib):
    """The RoPE-rotated K scratch is one cached buffer per (device, stream):
    calls on two streams in flight together, and a call that grows a stream's
    buffer between two smaller ones, give the bits of the same calls made one
    at a time."""
    import rdnattention

    shapes = [(1, 8, 2, 300, 128, True), (2, 8, 4, 900, 64, False), (1, 4, 1, 1500, 128, True)]
    cases = []
    for i, (b, hq, hkv, s, d, causal) in enumerate(shapes):
        q, k, v = seeded_inputs(40 + i, b, hq, hkv, s, s, d)
        cos, sin = oracle.rope_tables(s, d)
        cases.append((q.to(gpu), k.to(gpu), v.to(gpu), torch.from_numpy(cos).to(gpu),
                      torch.from_numpy(sin).to(gpu), causal))

    def run(c):
        q, k, v, cd, sd, causal = c
        return rdnattention.flash_attn(q, k, v, is_causal=causal, rot_cos=cd, rot_sin=sd)

    log("[cached scratch] one at a time")
    refs = []
    for c in cases:
        refs.append(run(c))
        torch.cuda.synchronize()
    rdnattention.trim_scratch()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    log("[cached scratch] two streams, growing buffers")
    outs = []
    for _ in range(3):
        with torch.cuda.stream(s1):
            outs.append((0, run(cases[0])))
            outs.append((2, run(cases[2])))  # grows s1's buffer
            outs.append((0, run(cases[0])))
        with torch.cuda.stream(s2):
            outs.append((1, run(cases[1])))
            outs.append((2, run(cases[2])))
    torch.cuda.synchronize()
    for i, o in outs:
        assert torch.equal(o, refs[i]), i
    for i, c in enumerate(cases):
        q, k, v, cd, sd, causal = c
        assert_f16_parity(refs[i].float().cpu().numpy(),
                          reference_f16(q.cpu(), k.cpu(), v.cpu(), causal, -1, cd.cpu().numpy(), sd.cpu().numpy()),
                          f"cached scratch {i}")
    rdnattention.trim_scratch()
