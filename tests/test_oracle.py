"""Pins the CPU oracle (oracle/attn_oracle.c) before anything is checked against it.

Every oracle function is checked against something other than its own formula:
a library routine (numpy's float16, torch SDPA with torch.tril/triu masks,
numpy int64 matmul, torch.round/clamp as the reference's quantisers call them),
a closed form (the causal pair count of tests/benchmark.py:77-88, V[0] for the
first causal row, the mean of visible V for constant scores), an invariant
(GQA == repeated K/V, channel permutation, RoPE relative position), or a
hand-written known-answer set (mask visibility from docs/api.md:150-165).
The reference ships no golden vectors or fixture files, so these are the pins.
"""
import numpy as np
import pytest
import torch

pytestmark = []


# --------------------------------------------------------------------------- #
# fp16 conversion vs numpy's float16 (library routine)
# --------------------------------------------------------------------------- #
def test_half_to_float_exhaustive(oracle_lib):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle_lib.half_to_float(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_matches_numpy(oracle_lib):
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        # exact ties between adjacent halves, normal and subnormal
        (np.arange(0, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -24),
        (np.float32(1.0) + (np.arange(0, 1024, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10)),
        np.array([65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1e-5, 6.0e-8, 2.98e-8, 0.0, -0.0, np.inf, -np.inf],
                 dtype=np.float32),
    ])
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([oracle_lib.float_to_half(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got, ref)


# --------------------------------------------------------------------------- #
# masks and work counting
# --------------------------------------------------------------------------- #
def _closed_form_causal_pairs(sq, sk):
    # tests/benchmark.py:77-88
    delta = sk - sq
    t = max(0, min(sk - delta, sq))
    return t * (delta + 1) + t * (t - 1) // 2 + (sq - t) * sk


@pytest.mark.parametrize("sq,sk", [(1, 1), (7, 7), (512, 512), (4096, 4096), (1, 300), (4, 300), (64, 300),
                                   (300, 64), (8192, 8192)])
def test_valid_pairs_causal_closed_form(oracle_lib, sq, sk):
    if sq > sk:
        # the reference's closed form assumes delta >= 0; rows above the cache see nothing
        delta = sk - sq
        expect = sum(max(0, min(i + delta, sk - 1) + 1) for i in range(sq))
    else:
        expect = _closed_form_causal_pairs(sq, sk)
    assert oracle_lib.valid_pairs(sq, sk, True, -1) == expect


def test_valid_pairs_known_workloads(oracle_lib):
    # the exact pair counts of the measured workloads
    assert oracle_lib.valid_pairs(512, 512, False, -1) == 262144
    assert oracle_lib.valid_pairs(4096, 4096, True, -1) == 8390656
    assert oracle_lib.valid_pairs(8192, 8192, True, -1) == 33558528
    assert oracle_lib.valid_pairs(1, 32768, False, -1) == 32768
    assert oracle_lib.valid_pairs(16384, 16384, False, 4096) == 62928896
    assert oracle_lib.valid_pairs(4096, 4096, False, 4096) == 12584960


@pytest.mark.parametrize("sq,sk,causal,window", [(5, 5, True, -1), (5, 9, True, 3), (9, 5, False, 4),
                                                 (6, 6, False, 1), (3, 10, False, 6), (10, 3, True, 2)])
def test_valid_pairs_brute_force(oracle_lib, sq, sk, causal, window):
    brute = sum(oracle_lib.visible(i, k, sq, sk, causal, window) for i in range(sq) for k in range(sk))
    assert oracle_lib.valid_pairs(sq, sk, causal, window) == brute


# Hand-written visibility sets from the reference's documented rules
# (docs/api.md:150-165): causal aligns to the end of the keys (delta = Sk - Sq,
# key k visible iff k <= q + delta); causal window w = the w keys ending at
# q + delta; non-causal window = |q + delta - k| <= w // 2.
KAT_VISIBILITY = [
    # (sq, sk, causal, window, {row: visible keys})
    (3, 3, True, -1, {0: [0], 1: [0, 1], 2: [0, 1, 2]}),
    (2, 4, True, -1, {0: [0, 1, 2], 1: [0, 1, 2, 3]}),  # delta = 2
    (4, 2, True, -1, {0: [], 1: [], 2: [0], 3: [0, 1]}),  # delta = -2: rows 0,1 see nothing
    (4, 4, True, 2, {0: [0], 1: [0, 1], 2: [1, 2], 3: [2, 3]}),
    (4, 4, False, 2, {0: [0, 1], 1: [0, 1, 2], 2: [1, 2, 3], 3: [2, 3]}),
    (4, 4, False, 3, {0: [0, 1], 1: [0, 1, 2], 2: [1, 2, 3], 3: [2, 3]}),  # w // 2 = 1
    (1, 5, False, 4, {0: [2, 3, 4]}),  # delta = 4, band [2, 6] clipped to [2, 4]
    (1, 5, True, -1, {0: [0, 1, 2, 3, 4]}),  # decode sees the whole cache
    (3, 3, False, 0, {0: [0, 1, 2], 1: [0, 1, 2], 2: [0, 1, 2]}),  # window 0 = off
]


@pytest.mark.parametrize("sq,sk,causal,window,expect", KAT_VISIBILITY)
def test_mask_known_answers_through_attention(oracle_lib, sq, sk, causal, window, expect):
    """Q = 0 gives equal weight to every visible key; V = one-hot(key) then
    reveals the visible set as the non-zero output columns (and 0 rows for
    rows that see nothing)."""
    d = 32
    q = np.zeros((1, 1, sq, d), np.float32)
    k = np.random.default_rng(1).standard_normal((1, 1, sk, d)).astype(np.float32)
    v = np.zeros((1, 1, sk, d), np.float32)
    for j in range(sk):
        v[0, 0, j, j] = 1.0
    out = oracle_lib.attention(q, k, v, causal=causal, window=window)[0, 0]
    for row, keys in expect.items():
        want = np.zeros(d, np.float32)
        if keys:
            want[keys] = 1.0 / len(keys)
        np.testing.assert_allclose(out[row], want, atol=1e-7, err_msg=f"row {row}")
        for kk in range(sk):
            assert oracle_lib.visible(row, kk, sq, sk, causal, window) == (kk in keys)


# --------------------------------------------------------------------------- #
# attention vs torch SDPA (library routine) with torch.tril/triu masks
# --------------------------------------------------------------------------- #
def _torch_mask(sq, sk, causal, window):
    delta = sk - sq
    ones = torch.ones(sq, sk, dtype=torch.bool)
    m = ones.clone()
    if causal:
        m &= torch.tril(ones, diagonal=delta)
    if window > 0:
        if causal:
            m &= torch.triu(ones, diagonal=delta - window + 1)
        else:
            hw = window // 2
            m &= torch.triu(ones, diagonal=delta - hw) & torch.tril(ones, diagonal=delta + hw)
    return m


SDPA_CASES = [
    # b, hq, hkv, sq, sk, d, causal, window
    (1, 2, 2, 33, 33, 32, False, -1),
    (2, 4, 2, 40, 40, 64, True, -1),
    (1, 4, 1, 17, 50, 64, True, -1),
    (1, 2, 2, 50, 17, 32, False, -1),
    (1, 2, 2, 64, 64, 64, False, 16),
    (1, 2, 2, 64, 64, 64, True, 9),
    (1, 6, 3, 5, 70, 96, False, 20),
    (1, 1, 1, 1, 100, 128, False, -1),
]


@pytest.mark.parametrize("b,hq,hkv,sq,sk,d,causal,window", SDPA_CASES)
def test_attention_vs_torch_sdpa(oracle_lib, b, hq, hkv, sq, sk, d, causal, window):
    g = torch.Generator().manual_seed(11)
    q = torch.randn(b, hq, sq, d, generator=g, dtype=torch.float64)
    k = torch.randn(b, hkv, sk, d, generator=g, dtype=torch.float64)
    v = torch.randn(b, hkv, sk, d, generator=g, dtype=torch.float64)
    mask = _torch_mask(sq, sk, causal, window)
    rows_ok = mask.any(dim=1)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q, k.repeat_interleave(hq // hkv, 1), v.repeat_interleave(hq // hkv, 1), attn_mask=mask)
    ref = torch.where(rows_ok[None, None, :, None], ref, torch.zeros_like(ref))  # SDPA gives NaN there
    got = oracle_lib.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=causal, window=window)
    # inputs were rounded to fp32 for the oracle; compare against fp64 SDPA on the same rounded inputs
    ref32 = torch.nn.functional.scaled_dot_product_attention(
        q.float().double(), k.float().double().repeat_interleave(hq // hkv, 1),
        v.float().double().repeat_interleave(hq // hkv, 1), attn_mask=mask)
    ref32 = torch.where(rows_ok[None, None, :, None], ref32, torch.zeros_like(ref32))
    np.testing.assert_allclose(got, ref32.numpy(), atol=2e-6, rtol=1e-5)
    assert torch.allclose(ref32, ref, atol=1e-5)


# --------------------------------------------------------------------------- #
# closed forms and invariants
# --------------------------------------------------------------------------- #
def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def test_first_causal_row_is_v0(oracle_lib):
    q, k, v = _rand((1, 2, 16, 64), 1), _rand((1, 2, 16, 64), 2), _rand((1, 2, 16, 64), 3)
    out = oracle_lib.attention(q, k, v, causal=True)
    np.testing.assert_array_equal(out[:, :, 0], v[:, :, 0])


def test_decode_causal_equals_noncausal(oracle_lib):
    q, k, v = _rand((2, 4, 1, 64), 4), _rand((2, 2, 77, 64), 5), _rand((2, 2, 77, 64), 6)
    a = oracle_lib.attention(q, k, v, causal=True)
    b = oracle_lib.attention(q, k, v, causal=False)
    np.testing.assert_array_equal(a, b)


def test_rows_without_keys_are_zero(oracle_lib):
    q, k, v = _rand((1, 1, 8, 32), 7), _rand((1, 1, 3, 32), 8), _rand((1, 1, 3, 32), 9)
    out = oracle_lib.attention(q, k, v, causal=True)  # delta = -5: rows 0..4 see nothing
    assert np.all(out[0, 0, :5] == 0.0)
    assert np.all(np.abs(out[0, 0, 5:]).sum(-1) > 0)


def test_zero_query_is_mean_of_visible_values(oracle_lib):
    k, v = _rand((1, 1, 20, 32), 10), _rand((1, 1, 20, 32), 11)
    q = np.zeros((1, 1, 20, 32), np.float32)
    out = oracle_lib.attention(q, k, v, causal=True)
    for i in range(20):
        np.testing.assert_allclose(out[0, 0, i], v[0, 0, : i + 1].astype(np.float64).mean(0), atol=1e-6)


def test_huge_window_is_no_window(oracle_lib):
    q, k, v = _rand((1, 2, 30, 32), 12), _rand((1, 2, 45, 32), 13), _rand((1, 2, 45, 32), 14)
    for causal in (False, True):
        a = oracle_lib.attention(q, k, v, causal=causal, window=4 * 45 + 10)
        b = oracle_lib.attention(q, k, v, causal=causal, window=-1)
        np.testing.assert_array_equal(a, b)


def test_gqa_equals_repeated_kv(oracle_lib):
    q, k, v = _rand((2, 8, 19, 64), 15), _rand((2, 2, 23, 64), 16), _rand((2, 2, 23, 64), 17)
    a = oracle_lib.attention(q, k, v, causal=True, window=7)
    b = oracle_lib.attention(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), causal=True, window=7)
    np.testing.assert_array_equal(a, b)


def test_common_channel_permutation_invariance(oracle_lib):
    q, k, v = _rand((1, 2, 25, 64), 18), _rand((1, 2, 25, 64), 19), _rand((1, 2, 25, 64), 20)
    perm = np.random.default_rng(21).permutation(64)
    a = oracle_lib.attention(q, k, v)
    b = oracle_lib.attention(q[..., perm], k[..., perm], v)
    np.testing.assert_allclose(a, b, atol=1e-6)


def test_brute_force_tiny_vs_numpy_softmax(oracle_lib):
    from scipy.special import softmax

    q, k, v = _rand((1, 1, 5, 32), 22), _rand((1, 1, 7, 32), 23), _rand((1, 1, 7, 32), 24)
    s = (q[0, 0].astype(np.float64) @ k[0, 0].astype(np.float64).T) / np.sqrt(32.0)
    ref = softmax(s, axis=-1) @ v[0, 0].astype(np.float64)
    np.testing.assert_allclose(oracle_lib.attention(q, k, v)[0, 0], ref, atol=1e-6)


def test_lse_output(oracle_lib):
    from scipy.special import logsumexp

    q, k, v = _rand((1, 1, 6, 32), 25), _rand((1, 1, 9, 32), 26), _rand((1, 1, 9, 32), 27)
    _, lse = oracle_lib.attention(q, k, v, return_lse=True)
    s = (q[0, 0].astype(np.float64) @ k[0, 0].astype(np.float64).T) / np.sqrt(32.0)
    np.testing.assert_allclose(lse[0, 0], logsumexp(s, axis=-1), rtol=1e-6)


# --------------------------------------------------------------------------- #
# RoPE
# --------------------------------------------------------------------------- #
def test_rope_known_answer(oracle_lib):
    # docs/api.md:92-93: channels 2i and 2i+1 rotate together by the angle in column i
    d = 8
    x = np.zeros((1, 3, d), np.float32)
    x[0, :, 2] = 1.0  # pair i = 1, first element
    cos = np.array([[1, 1, 1, 1], [0.5, 0.25, 1, 1], [0, -1, 1, 1]], np.float32)
    sin = np.array([[0, 0, 0, 0], [0.75, 0.125, 0, 0], [1, 0.5, 0, 0]], np.float32)
    y = oracle_lib.rope(x, cos, sin, round_f16=False)
    # (a, b) = (1, 0) -> (a c - b s, a s + b c) = (c, s) at column 1
    np.testing.assert_array_equal(y[0, :, 2], cos[:, 1])
    np.testing.assert_array_equal(y[0, :, 3], sin[:, 1])
    assert np.all(y[0, :, [0, 1, 4, 5, 6, 7]] == 0)


def test_rope_relative_position_property(oracle_lib):
    """<R(m) q, R(n) k> depends only on m - n when the tables are true angles."""
    d = 64
    cos, sin = oracle_lib.rope_tables(64, d)
    rng = np.random.default_rng(30)
    qv, kv = rng.standard_normal(d).astype(np.float32), rng.standard_normal(d).astype(np.float32)
    q = np.tile(qv, (1, 64, 1))
    k = np.tile(kv, (1, 64, 1))
    qr = oracle_lib.rope(q, cos, sin, round_f16=False)[0].astype(np.float64)
    kr = oracle_lib.rope(k, cos, sin, round_f16=False)[0].astype(np.float64)
    for off in (0, 3, 11):
        dots = [qr[m] @ kr[m - off] for m in range(off, 40)]
        np.testing.assert_allclose(dots, dots[0], atol=2e-3)


def test_rope_rotate_half_equivalence(oracle_lib):
    """Interleaved RoPE on permuted channels == HF-style rotate-half RoPE, permuted
    (x*cos + rotate_half(x)*sin with cos/sin repeated over both halves)."""
    d = 32
    cos, sin = oracle_lib.rope_tables(12, d)
    x = _rand((1, 12, d), 31)
    perm = oracle_lib.rotate_half_perm(d)
    inter = oracle_lib.rope(x[..., perm], cos, sin, round_f16=False)
    c2 = np.concatenate([cos, cos], -1).astype(np.float64)
    s2 = np.concatenate([sin, sin], -1).astype(np.float64)
    xd = x.astype(np.float64)
    rot = np.concatenate([-xd[..., d // 2:], xd[..., : d // 2]], -1)
    half = xd * c2 + rot * s2
    np.testing.assert_allclose(inter, half[..., perm], atol=1e-5)


def test_rope_fp16_rounding_flag(oracle_lib):
    cos, sin = oracle_lib.rope_tables(20, 64)
    x = _rand((2, 20, 64), 32)
    a = oracle_lib.rope(x, cos, sin, round_f16=False)
    b = oracle_lib.rope(x, cos, sin, round_f16=True)
    np.testing.assert_array_equal(b, a.astype(np.float16).astype(np.float32))


# --------------------------------------------------------------------------- #
# INT8
# --------------------------------------------------------------------------- #
def test_int8_scores_vs_numpy_int64(oracle_lib):
    rng = np.random.default_rng(40)
    qi = rng.integers(-127, 128, (2, 4, 9, 128), dtype=np.int8)
    ki = rng.integers(-127, 128, (2, 2, 13, 128), dtype=np.int8)
    qi[0, 0, 0] = 127
    ki[0, 0, 0] = 127  # the extreme |sum| = 127^2 * 128
    s = oracle_lib.int8_scores(qi, ki)
    ref = np.einsum("bhqd,bhkd->bhqk", qi.astype(np.int64), np.repeat(ki, 2, axis=1).astype(np.int64))
    assert np.array_equal(s.astype(np.int64), ref)
    assert s[0, 0, 0, 0] == 127 * 127 * 128


def test_int8_constant_scores_give_mean_v(oracle_lib):
    """Q = 0: every p = 1 -> pq = 127 exactly -> O = mean(V) * v_scale."""
    rng = np.random.default_rng(41)
    qi = np.zeros((1, 2, 10, 64), np.int8)
    ki = rng.integers(-127, 128, (1, 2, 150, 64), dtype=np.int8)
    vi = rng.integers(-127, 128, (1, 2, 150, 64), dtype=np.int8)
    out = oracle_lib.attention_int8(qi, ki, vi, 0.01, 0.02, 0.5, block_n=64)
    ref = vi.astype(np.float64).mean(axis=2, keepdims=True) * 0.5
    np.testing.assert_allclose(out, np.broadcast_to(ref, out.shape), rtol=1e-5, atol=1e-6)


def _int8_inputs(seed, b, hq, hkv, sq, sk, d):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((b, hq, sq, d)).astype(np.float32)
    k = rng.standard_normal((b, hkv, sk, d)).astype(np.float32)
    v = rng.standard_normal((b, hkv, sk, d)).astype(np.float32)
    return q, k, v


def test_int8_single_block_matches_gate_flavour(oracle_lib):
    """With every key in one block the running max IS the global max, so the
    kernel-exact emulation must equal the gate's global-max flavour up to the
    fp32 vs fp64 arithmetic (rare lround ties at most)."""
    q, k, v = _int8_inputs(42, 1, 4, 4, 20, 60, 64)
    qi, qs = oracle_lib.quant_pertoken(q)
    ki, ks = oracle_lib.quant_pertoken(k)
    vi, vs = oracle_lib.quant_pertensor(v)
    blk = oracle_lib.attention_int8(qi, ki, vi, qs, ks, vs, block_n=64)
    gate = oracle_lib.attention_int8_gate(qi * qs[..., None], ki * ks[..., None], vi.astype(np.float32) * vs)
    diff = np.abs(blk - gate)
    assert np.median(diff) < 1e-6
    assert diff.max() < 2e-2 * np.abs(gate).max()


def test_int8_quantised_p_is_lround_of_127p(oracle_lib):
    """One 64-key block and a one-hot V (row j = e_j) make the output row the
    quantised P: o_ij = pq_ij * v_scale / (127 l_i).  The row's best key has
    pq = 127, so pq_ij = 127 o_ij / max_j o_ij must be round(127 p_ij) with
    p = 2^(s - max s), s = S qs ks scale log2(e) evaluated in float64 from
    the exact int32 scores -- except within fp32 rounding of a tie at
    k + 1/2.  A floor for the rounding, a 128 scale or a P taken against
    another maximum fails (src/rdna/fa2_forward_int8qk.hip:301, :335)."""
    rng = np.random.default_rng(7)
    b, h, sq, sk, d = 1, 2, 256, 64, 64
    qi = rng.integers(-127, 128, (b, h, sq, d), dtype=np.int8)
    ki = rng.integers(-127, 128, (b, h, sk, d), dtype=np.int8)
    vi = np.zeros((b, h, sk, d), np.int8)
    vi[:, :, np.arange(sk), np.arange(sk)] = 1
    qs = rng.uniform(0.012, 0.028, (b, h, sq)).astype(np.float32)
    ks = rng.uniform(0.012, 0.028, (b, h, sk)).astype(np.float32)
    o = oracle_lib.attention_int8(qi, ki, vi, qs, ks, 127.0).astype(np.float64)
    y = 127.0 * o / o.max(axis=-1, keepdims=True)
    pq = np.rint(y)
    assert np.abs(y - pq).max() < 1e-4
    s = oracle_lib.int8_scores(qi, ki).astype(np.float64) * qs[..., None] * ks[:, :, None, :]
    s *= d ** -0.5 * np.log2(np.e)
    want = 127.0 * np.exp2(s - s.max(axis=-1, keepdims=True))
    off = pq != np.rint(want)
    assert np.count_nonzero(pq) > 0.3 * pq.size  # P spans the quantiser's range
    assert np.all(np.abs(want[off] - np.floor(want[off]) - 0.5) < 1e-4)


def test_int8_blockwise_close_to_fp_attention(oracle_lib):
    """The quantised scheme approximates fp attention to the reference gate's bar
    (rel_rms < 5e-2, tests/hip_forward_int8qk_gate.hip:248)."""
    q, k, v = _int8_inputs(43, 1, 4, 2, 150, 300, 128)
    qi, qs = oracle_lib.quant_pertoken(q)
    ki, ks = oracle_lib.quant_pertoken(k)
    vi, vch = oracle_lib.quant_perchannel(v)
    out = oracle_lib.attention_int8(qi, ki, vi, qs, ks, 1.0, causal=True) * np.repeat(vch, 2, axis=1)[:, :, None, :]
    ref = oracle_lib.attention(q, k, v, causal=True)
    rel = np.sqrt(((out - ref) ** 2).mean() / (ref ** 2).mean())
    assert rel < 5e-2


def test_int8_blockwise_depends_on_running_max(oracle_lib):
    """A planted change in block size must change the result (the running max
    is part of the scheme), while block sizes >= Sk all agree exactly."""
    q, k, v = _int8_inputs(44, 1, 2, 2, 30, 200, 64)
    qi, qs = oracle_lib.quant_pertoken(q)
    ki, ks = oracle_lib.quant_pertoken(k)
    vi, vs = oracle_lib.quant_pertensor(v)
    a = oracle_lib.attention_int8(qi, ki, vi, qs, ks, vs, block_n=64)
    b = oracle_lib.attention_int8(qi, ki, vi, qs, ks, vs, block_n=32)
    c = oracle_lib.attention_int8(qi, ki, vi, qs, ks, vs, block_n=256)
    d = oracle_lib.attention_int8(qi, ki, vi, qs, ks, vs, block_n=512)
    assert not np.array_equal(a, b)
    np.testing.assert_array_equal(c, d)


def _vtoken_exact_inputs(seed, b, hq, hkv, sq, sk, d):
    """Per-token V inputs whose dequantised rows are exact integers: w in
    [-31, 31], vs in {1, 2, 4} per (batch, kv head, row), so w * vs is an int8
    value and fp16(w * vs) = w * vs."""
    rng = np.random.default_rng(seed)
    qi = rng.integers(-127, 128, (b, hq, sq, d), dtype=np.int8)
    ki = rng.integers(-127, 128, (b, hkv, sk, d), dtype=np.int8)
    w = rng.integers(-31, 32, (b, hkv, sk, d), dtype=np.int8)
    vs = rng.choice(np.array([1.0, 2.0, 4.0], np.float32), size=(b, hkv, sk))
    v_full = (w.astype(np.int32) * vs[..., None].astype(np.int32)).astype(np.int8)
    return qi, ki, w, vs, v_full


def test_int8_vtoken_exact_rows_equal_per_tensor_path(oracle_lib):
    """Per-token V scales that dequantise to exact integers must give exactly
    the per-tensor result on the pre-multiplied V: pins the row indexing of
    v_token per (batch, kv head, key) and the sum itself (a wrong row, head
    or batch offset would mix the {1, 2, 4} factors)."""
    qi, ki, w, vs, v_full = _vtoken_exact_inputs(61, 2, 4, 2, 40, 150, 64)
    a = oracle_lib.attention_int8(qi, ki, w, 0.004, 0.006, 1.0, causal=True, v_token=vs)
    b = oracle_lib.attention_int8(qi, ki, v_full, 0.004, 0.006, 1.0, causal=True)
    np.testing.assert_array_equal(a, b)
    c = oracle_lib.attention_int8(qi, ki, w, 0.004, 0.006, 1.0, causal=True, v_token=vs[:, ::-1].copy())
    assert not np.array_equal(a, c)  # the kv heads' scales swapped


def test_int8_vtoken_ones_and_constant_power_of_two(oracle_lib):
    """v_token = 1 is the per-tensor path with v_scale 1; v_token = 2^-3 is
    v_scale = 2^-3 (both products exact)."""
    rng = np.random.default_rng(62)
    qi = rng.integers(-127, 128, (1, 2, 30, 128), dtype=np.int8)
    ki = rng.integers(-127, 128, (1, 1, 90, 128), dtype=np.int8)
    vi = rng.integers(-127, 128, (1, 1, 90, 128), dtype=np.int8)
    ones = np.ones((1, 1, 90), np.float32)
    base = oracle_lib.attention_int8(qi, ki, vi, 0.01, 0.01, 1.0, window=40)
    np.testing.assert_array_equal(oracle_lib.attention_int8(qi, ki, vi, 0.01, 0.01, 1.0, window=40, v_token=ones),
                                  base)
    np.testing.assert_array_equal(
        oracle_lib.attention_int8(qi, ki, vi, 0.01, 0.01, 1.0, window=40, v_token=ones * 0.125),
        oracle_lib.attention_int8(qi, ki, vi, 0.01, 0.01, 0.125, window=40))


@pytest.mark.parametrize("vs0", [1.0e6, 1.0e-7])
def test_int8_vtoken_extreme_scales(oracle_lib, vs0):
    """One V row with a scale far outside the usual range: 1e6 drives v * vs
    beyond fp16 (it saturates to +-65504, never inf), 1e-7 into fp16
    subnormals.  Causal row 0 sees key 0 only, so its output is v'_0 itself:
    checked against numpy's fp16 rounding of the saturated fp32 product.
    Rows that cannot see key 0 (window 2: |i - j| <= 1) are bit-identical to a
    run with vs_0 = 1, and nothing is NaN or infinite."""
    rng = np.random.default_rng(64)
    sq = sk = 24
    qi = rng.integers(-127, 128, (1, 2, sq, 64), dtype=np.int8)
    ki = rng.integers(-127, 128, (1, 1, sk, 64), dtype=np.int8)
    vi = rng.integers(-127, 128, (1, 1, sk, 64), dtype=np.int8)
    vi[0, 0, 0, :8] = 127
    vi[0, 0, 0, 8:16] = -127
    vt = rng.uniform(0.01, 0.03, (1, 1, sk)).astype(np.float32)
    vt[0, 0, 0] = vs0
    out = oracle_lib.attention_int8(qi, ki, vi, 0.01, 0.01, 1.0, causal=True, v_token=vt)
    assert np.isfinite(out).all()
    want = np.clip(vi[0, 0, 0].astype(np.float32) * np.float32(vs0), -65504, 65504).astype(np.float16)
    np.testing.assert_array_equal(out[0, :, 0], np.broadcast_to(want.astype(np.float32), (2, 64)))
    w = oracle_lib.attention_int8(qi, ki, vi, 0.01, 0.01, 1.0, window=2, v_token=vt)
    vt1 = vt.copy()
    vt1[0, 0, 0] = 1.0
    w1 = oracle_lib.attention_int8(qi, ki, vi, 0.01, 0.01, 1.0, window=2, v_token=vt1)
    assert np.isfinite(w).all()
    np.testing.assert_array_equal(w[:, :, 2:], w1[:, :, 2:])
    assert not np.array_equal(w[:, :, :2], w1[:, :, :2])


def test_int8_vtoken_close_to_fp_attention(oracle_lib):
    """Per-token V quantisation approximates fp attention to the reference
    gate's bar (rel_rms < 5e-2)."""
    q, k, v = _int8_inputs(63, 1, 4, 2, 150, 300, 128)
    qi, qs = oracle_lib.quant_pertoken(q)
    ki, ks = oracle_lib.quant_pertoken(k)
    vi, vt = oracle_lib.quant_pertoken(v)
    out = oracle_lib.attention_int8(qi, ki, vi, qs, ks, 1.0, causal=True, v_token=vt)
    ref = oracle_lib.attention(q, k, v, causal=True)
    rel = np.sqrt(((out - ref) ** 2).mean() / (ref ** 2).mean())
    assert rel < 5e-2


# --------------------------------------------------------------------------- #
# quantisers vs the torch calls the reference makes (rdnattention/__init__.py)
# --------------------------------------------------------------------------- #
def _torch_per_token(x):
    # rdnattention/__init__.py:335-339
    x = x.float()
    s = x.abs().amax(dim=-1, keepdim=True) / 127.0
    s = torch.where(s == 0, torch.ones_like(s), s)
    return torch.clamp(torch.round(x / s), -127, 127).to(torch.int8), s.squeeze(-1).contiguous()


def _torch_per_channel_v(v):
    # rdnattention/__init__.py:320-324
    v = v.float()
    vc = v.abs().amax(dim=-2, keepdim=True) / 127.0
    vc = torch.where(vc == 0, torch.ones_like(vc), vc)
    return torch.clamp(torch.round(v / vc), -127, 127).to(torch.int8), vc.squeeze(-2)


def _torch_per_tensor(x):
    # rdnattention/__init__.py:313-316
    s = x.abs().max().item() / 127.0
    s = s if s != 0.0 else 1.0
    return torch.clamp(torch.round(x / s), -127, 127).to(torch.int8), s


def test_quant_pertoken_vs_torch(oracle_lib):
    g = torch.Generator().manual_seed(50)
    x = torch.randn(3, 4, 33, 64, generator=g)
    x[0, 0, 0] = 0.0  # zero row -> scale 1
    # exact ties: row max 127 -> scale 1, values k + 0.5
    x[0, 0, 1] = torch.arange(64).float() - 31.5
    x[0, 0, 1, 0] = 127.0
    qi, s = oracle_lib.quant_pertoken(x.numpy())
    tq, ts = _torch_per_token(x)
    assert np.array_equal(qi, tq.numpy())
    assert np.array_equal(s, ts.numpy())


def test_quant_perchannel_vs_torch(oracle_lib):
    g = torch.Generator().manual_seed(51)
    v = torch.randn(2, 3, 40, 32, generator=g)
    v[0, 0, :, 5] = 0.0
    vi, vch = oracle_lib.quant_perchannel(v.numpy())
    tq, tc = _torch_per_channel_v(v)
    assert np.array_equal(vi, tq.numpy())
    assert np.array_equal(vch, tc.numpy())


def test_quant_pertensor_vs_torch(oracle_lib):
    g = torch.Generator().manual_seed(52)
    x = torch.randn(2, 2, 20, 64, generator=g)
    qi, s = oracle_lib.quant_pertensor(x.numpy())
    tq, ts = _torch_per_tensor(x)
    assert np.float32(ts) == np.float32(s)
    assert np.array_equal(qi, tq.numpy())


# --------------------------------------------------------------------------- #
# the reference gates' LCG (tests/hip_forward_gate.hip:31-37)
# --------------------------------------------------------------------------- #
def test_lcg_stream(oracle_lib):
    s = 12345
    want = []
    for _ in range(5):
        s = (s * 1664525 + 1013904223) % (1 << 32)
        want.append(((s >> 16) & 4095) / 4096.0 - 0.5)
    got = oracle_lib.Lcg(12345).fill((5,), 0)
    np.testing.assert_array_equal(got, np.array(want, np.float32))
    g2 = oracle_lib.Lcg(424242)
    a = g2.fill((2,), 1)
    s = 424242
    vals = []
    for _ in range(6):
        s = (s * 1664525 + 1013904223) % (1 << 32)
        vals.append(np.float32(((s >> 16) & 4095) / 4096.0 - 0.5))
    np.testing.assert_array_equal(a, np.array([(vals[0] + vals[1] + vals[2]) / np.float32(3),
                                               (vals[3] + vals[4] + vals[5]) / np.float32(3)], np.float32))
