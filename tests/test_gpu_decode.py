"""Split-K decode path on the GPU against the CPU oracle.

The reference has no split-K kernel (docs/api.md:203-204); its decode shapes
run through the same FP16 entry point, so the bar is the FP16 one: max-abs
<= 2e-3, mean-abs <= 2e-4 and rel_rms < 5e-3 against the oracle on the same
inputs, for every mask mode, GQA ratio and stride layout the entry point
accepts.  The prefill kernel is run on the same inputs as a second path.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import assert_f16_parity, forward_raw, log, reference_f16, seeded_inputs

pytestmark = pytest.mark.gpu

PATH_PREFILL, PATH_SPLITK = 1, 2

# b, hq, hkv, sq, sk, d, causal, window, rope
CASES = [
    (2, 8, 2, 1, 1000, 64, False, -1, False),
    (2, 8, 2, 4, 3000, 128, False, -1, False),
    (1, 32, 8, 1, 32768, 128, False, -1, False),
    (1, 32, 8, 4, 8192, 128, False, -1, False),
    (1, 32, 1, 1, 5000, 128, False, -1, False),   # MQA, 32 columns
    (1, 16, 2, 4, 2048, 64, False, -1, False),    # ratio 8 x Sq 4 = 32 columns
    (2, 4, 4, 3, 777, 32, False, -1, False),
    (2, 8, 2, 4, 3000, 128, True, -1, False),     # causal decode: last keys masked per row
    (1, 8, 2, 4, 3000, 128, True, 700, False),    # causal window
    (1, 8, 2, 2, 3000, 64, False, 900, False),    # two-sided window
    (1, 8, 2, 1, 2500, 128, False, -1, True),     # RoPE (Q row 0, K rows 0..Sk-1)
    (1, 4, 2, 5, 40, 64, True, -1, False),        # short: fewer keys than one wave round
]


@pytest.mark.parametrize("case", CASES, ids=[f"b{c[0]}h{c[1]}kv{c[2]}q{c[3]}k{c[4]}d{c[5]}c{int(c[6])}w{c[7]}r{int(c[8])}"
                                             for c in CASES])
def test_splitk_vs_oracle(gpu, oracle_lib, case):
    b, hq, hkv, sq, sk, d, causal, window, rope = case
    log(f"[splitk] {case}")
    q, k, v = seeded_inputs(21, b, hq, hkv, sq, sk, d)
    cos = sin = None
    if rope:
        cos, sin = oracle.rope_tables(max(sq, sk), d)
    ref = reference_f16(q, k, v, causal, window, cos, sin)
    cd = torch.from_numpy(cos).to(gpu) if rope else None
    sd = torch.from_numpy(sin).to(gpu) if rope else None
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    outs = {}
    for path in (PATH_SPLITK, PATH_PREFILL, 0):
        o = torch.full_like(qd, float("nan"))
        assert forward_raw(qd, kd, vd, o, causal, window, cd, sd, path=path) == 0
        outs[path] = o
    torch.cuda.synchronize()
    for path, o in outs.items():
        assert_f16_parity(o.float().cpu().numpy(), ref, f"path{path}")


def test_splitk_strided_cache_views(gpu, oracle_lib):
    """K/V sliced from one [B, S, 2, Hkv, D] cache (the decode benchmark's layout)."""
    g = torch.Generator().manual_seed(3)
    b, hq, hkv, sq, sk, d = 2, 16, 4, 4, 4096, 128
    buf = torch.randn(b, sk, 2, hkv, d, generator=g).half()
    q = torch.randn(b, hq, sq, d, generator=g).half()
    bd = buf.to(gpu)
    kv_k = bd[:, :, 0].transpose(1, 2)
    kv_v = bd[:, :, 1].transpose(1, 2)
    o1 = torch.empty(b, hq, sq, d, dtype=torch.float16, device=gpu)
    o2 = torch.empty_like(o1)
    qd = q.to(gpu)
    assert forward_raw(qd, kv_k, kv_v, o1, path=PATH_SPLITK) == 0
    assert forward_raw(qd, kv_k.contiguous(), kv_v.contiguous(), o2, path=PATH_SPLITK) == 0
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    ref = reference_f16(q, buf[:, :, 0].transpose(1, 2), buf[:, :, 1].transpose(1, 2), False, -1)
    assert_f16_parity(o1.float().cpu().numpy(), ref, "strided_cache")


def test_splitk_rows_without_keys(gpu):
    """Causal with Sq > Sk through split-K: rows above the cache write 0."""
    q, k, v = seeded_inputs(5, 1, 4, 4, 8, 3, 64)
    out = torch.full_like(q, 7.0, device=gpu)
    assert forward_raw(q.to(gpu), k.to(gpu), v.to(gpu), out, causal=True, path=PATH_SPLITK) == 0
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    assert np.all(o[:, :, :5] == 0)
    assert_f16_parity(o, reference_f16(q, k, v, True, -1), "no_keys")


def test_splitk_unsupported_shape_is_rejected(gpu):
    q = torch.zeros(1, 8, 9, 128, dtype=torch.float16, device=gpu)  # ratio 4 x 9 rows = 36 columns > 32
    k = torch.zeros(1, 2, 100, 128, dtype=torch.float16, device=gpu)
    out = torch.empty_like(q)
    import rdnattention

    assert forward_raw(q, k, k, out, path=PATH_SPLITK) == -3
    assert "split-K" in rdnattention.last_error()
    assert forward_raw(q, k, k, out, path=0) == 0  # auto falls back to the prefill kernel
