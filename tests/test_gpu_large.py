"""Maximum sizes: K/V (and Q/O) tensors of 17 x 2^27 fp16 elements (4.25 GiB
each), so the element offsets of the last head exceed 2^31 (its byte offsets
2^32) and every base address must be computed in 64 bits. The checked slices (first/last heads, the last rows)
carry the largest offsets; the inputs are generated on the GPU and only those
slices are copied to the CPU oracle."""
import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import assert_f16_parity, forward_raw, log

pytestmark = pytest.mark.gpu

S_BIG = 1 << 20  # rows per head; 17 heads x 2^20 rows x 128 > 2^31 elements per tensor
H_BIG = 17


def _randn(gpu, shape, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    return torch.randn(shape, generator=g, device=gpu, dtype=torch.float16)


def test_decode_kv_beyond_2g_elements(gpu, oracle_lib):
    log("[large] split-K decode, K/V [1, 17, 2^20, 128] fp16 (4.25 GiB each)")
    hkv, d = H_BIG, 128
    k = _randn(gpu, (1, hkv, S_BIG, d), 40)
    v = _randn(gpu, (1, hkv, S_BIG, d), 41)
    q = _randn(gpu, (1, hkv, 1, d), 42)
    o = torch.full_like(q, float("nan"))
    assert forward_raw(q, k, v, o, path=2) == 0
    torch.cuda.synchronize()
    for h in (0, 8, hkv - 1):
        ref = oracle.attention(q[:, h:h + 1].float().cpu().numpy(), k[:, h:h + 1].float().cpu().numpy(),
                               v[:, h:h + 1].float().cpu().numpy())
        assert_f16_parity(o[:, h:h + 1].float().cpu().numpy(), ref, f"decode head {h}")
    del q, k, v, o
    torch.cuda.empty_cache()


def test_windowed_prefill_beyond_2g_elements(gpu, oracle_lib):
    """Two-sided window of 64 (|q - k| <= 32) over S = 2^20 rows: the last 200
    rows of a head see keys S - 232 .. S - 1 only, so the oracle runs on that
    slice, aligned to the end (its delta = Sk' - Sq' = 32 puts row i of the
    slice at global distance 32 + i - j from slice key j)."""
    log("[large] windowed prefill, Q/K/V/O [1, 17, 2^20, 128] fp16 (4.25 GiB each)")
    h, d, w, n = H_BIG, 128, 64, 200
    q = _randn(gpu, (1, h, S_BIG, d), 43)
    k = _randn(gpu, (1, h, S_BIG, d), 44)
    v = _randn(gpu, (1, h, S_BIG, d), 45)
    o = torch.full_like(q, float("nan"))
    assert forward_raw(q, k, v, o, window=w, path=1) == 0
    torch.cuda.synchronize()
    lo_k = S_BIG - n - w // 2
    for hh in (0, h - 1):
        ref = oracle.attention(q[:, hh:hh + 1, S_BIG - n:].float().cpu().numpy(),
                               k[:, hh:hh + 1, lo_k:].float().cpu().numpy(),
                               v[:, hh:hh + 1, lo_k:].float().cpu().numpy(), window=w)
        assert_f16_parity(o[:, hh:hh + 1, S_BIG - n:].float().cpu().numpy(), ref, f"window head {hh}")
    del q, k, v, o
    torch.cuda.empty_cache()
