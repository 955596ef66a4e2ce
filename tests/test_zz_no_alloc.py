"""rdna_attention_forward_noalloc: the entry point that allocates nothing.

Its scratch (the RoPE-rotated K copy, the split-K partials) comes from the
library's static per-device array instead of stream-ordered allocations, so
its results must be bit-identical to rdna_attention_forward's on the same
inputs.  Checked through the C ABI on two calls in a row, the second with a
smaller input (the array keeps the first call's contents), for each scratch
user and for both together; a call needing more than the array's 64 MiB is
refused with -3 before anything is launched; and one result is checked
against the CPU oracle as well.
"""
import pytest
import torch

import oracle
from tests.gpu_util import assert_f16_parity, lib, log, reference_f16, stream_ptr

pytestmark = pytest.mark.gpu

LIMIT = 64 << 20


def _call(fn, q, k, v, out, causal=False, window=-1, cos=None, sin=None):
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    qs, ks, vs, os_ = q.stride(), k.stride(), v.stride(), out.stride()
    return fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
              cos.data_ptr() if cos is not None else None, sin.data_ptr() if sin is not None else None,
              qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os_[0], os_[1], os_[2],
              b, hq, hkv, sq, sk, d, d ** -0.5, 1 if causal else 0, 1 if cos is not None else 0, int(window),
              stream_ptr())


def _inputs(gpu, seed, b, hq, hkv, sq, sk, d, rope, cache):
    g = torch.Generator(device=gpu).manual_seed(seed)
    q = torch.randn(b, hq, sq, d, device=gpu, generator=g).half()
    if cache:  # K/V views of one [B, S, 2, Hkv, D] cache
        c = torch.randn(b, sk, 2, hkv, d, device=gpu, generator=g).half()
        k, v = c[:, :, 0].transpose(1, 2), c[:, :, 1].transpose(1, 2)
    else:
        k = torch.randn(b, hkv, sk, d, device=gpu, generator=g).half()
        v = torch.randn(b, hkv, sk, d, device=gpu, generator=g).half()
    cos = sin = None
    if rope:
        ct, st = oracle.rope_tables(max(sq, sk), d)
        cos, sin = torch.from_numpy(ct).to(gpu), torch.from_numpy(st).to(gpu)
    return q, k, v, cos, sin


# name, (b, hq, hkv, sq, sk, d, causal, rope, cache) for the first and the second (smaller) call
CASES = [
    ("rope_prefill", (2, 8, 2, 300, 300, 128, True, True, False), (1, 4, 1, 77, 77, 128, True, True, False)),
    ("splitk_decode", (4, 32, 8, 1, 8192, 128, False, False, True), (2, 16, 4, 4, 3000, 128, False, False, True)),
    ("rope_splitk", (2, 16, 4, 2, 5000, 64, True, True, True), (1, 8, 2, 1, 1500, 64, True, True, False)),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_forward_twice(gpu, case):
    name, first, second = case
    L = lib()
    for call, (b, hq, hkv, sq, sk, d, causal, rope, cache) in enumerate((first, second)):
        log(f"[noalloc] {name} call {call}: b{b} hq{hq} hkv{hkv} sq{sq} sk{sk} d{d} rope={rope} cache={cache}")
        q, k, v, cos, sin = _inputs(gpu, 90 + call, b, hq, hkv, sq, sk, d, rope, cache)
        got = torch.full_like(q, float("nan"))
        want = torch.full_like(q, float("nan"))
        assert _call(L.rdna_attention_forward_noalloc, q, k, v, got, causal, -1, cos, sin) == 0, \
            L.rdna_get_error()
        assert _call(L.rdna_attention_forward, q, k, v, want, causal, -1, cos, sin) == 0, L.rdna_get_error()
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"{name} call {call}"


def test_noalloc_vs_oracle(gpu, oracle_lib):
    log("[noalloc] RoPE split-K decode vs the CPU oracle")
    q, k, v, cos, sin = _inputs(gpu, 95, 2, 8, 2, 3, 2000, 128, True, False)
    out = torch.full_like(q, float("nan"))
    assert _call(lib().rdna_attention_forward_noalloc, q, k, v, out, True, -1, cos, sin) == 0
    torch.cuda.synchronize()
    ref = reference_f16(q.cpu(), k.cpu(), v.cpu(), True, -1, cos.cpu().numpy(), sin.cpu().numpy())
    assert_f16_parity(out.float().cpu().numpy(), ref, "noalloc decode")


def test_noalloc_refuses_oversize_scratch(gpu):
    """A RoPE call whose rotated K copy alone is 128 MiB: -3 with the byte
    counts in the error, and the output untouched (nothing launched)."""
    log("[noalloc] 128 MiB of scratch requested: refused")
    q, k, v, cos, sin = _inputs(gpu, 96, 1, 16, 16, 64, 16384, 256, True, False)
    assert 16 * 16384 * 256 * 2 > LIMIT
    out = torch.full_like(q, float("nan"))
    L = lib()
    assert _call(L.rdna_attention_forward_noalloc, q, k, v, out, False, -1, cos, sin) == -3
    assert b"bytes of scratch" in L.rdna_get_error()
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
    del q, k, v, out
    torch.cuda.empty_cache()


def test_noalloc_makes_no_allocation(gpu):
    """After rdna_scratch_trim, calls of the no-allocation entry point that
    need both scratch buffers (RoPE-rotated K and split-K partials) leave the
    library's scratch cache empty and make no allocator call, while the
    allocating entry point on the same inputs does cache its buffers."""
    import rdnattention

    log("[noalloc] no cache entry and no allocator call after trim")
    L = lib()
    dev = torch.cuda.current_device()
    q, k, v, cos, sin = _inputs(gpu, 97, 2, 16, 4, 2, 5000, 64, True, True)
    out = torch.empty_like(q)
    torch.cuda.synchronize()
    rdnattention.trim_scratch()
    before = rdnattention.scratch_stats(dev)
    assert before["entries"] == 0 and before["cached_bytes"] == 0
    for _ in range(3):
        assert _call(L.rdna_attention_forward_noalloc, q, k, v, out, True, -1, cos, sin) == 0, L.rdna_get_error()
    torch.cuda.synchronize()
    after = rdnattention.scratch_stats(dev)
    assert after == before, (before, after)
    # the allocating entry point on the same call takes (and caches) two buffers
    assert _call(L.rdna_attention_forward, q, k, v, out, True, -1, cos, sin) == 0, L.rdna_get_error()
    torch.cuda.synchronize()
    cached = rdnattention.scratch_stats(dev)
    assert cached["entries"] == 2 and cached["allocations"] == before["allocations"] + 2, cached
    rdnattention.trim_scratch()
