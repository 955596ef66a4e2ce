"""The scratch cache of rdna_attention_forward: no allocator call and no host
wait once a stream is warm, growth that does not block the host, and a
per-device cap over all streams.

The reference allocates nothing (src/c_api.hpp:3-6).  The library's RoPE and
split-K paths need scratch; it is cached per (device, stream, use).  These
tests drive the C ABI on three streams with preallocated tensors, so that the
only device allocations in the measured regions are the library's own, and
read its counters through rdna_scratch_stats.
"""
import time

import pytest
import torch

import oracle
from tests.gpu_util import forward_raw, log

pytestmark = pytest.mark.gpu


def _inputs(gpu, seed, b, hq, hkv, sq, sk, d):
    g = torch.Generator(device=gpu).manual_seed(seed)
    q = torch.randn(b, hq, sq, d, device=gpu, generator=g).half()
    k = torch.randn(b, hkv, sk, d, device=gpu, generator=g).half()
    v = torch.randn(b, hkv, sk, d, device=gpu, generator=g).half()
    ct, st = oracle.rope_tables(max(sq, sk), d)
    return q, k, v, torch.from_numpy(ct).to(gpu), torch.from_numpy(st).to(gpu)


# (b, hq, hkv, sq, sk, d, causal): RoPE prefill (rotated K) and RoPE split-K
# decode (rotated K + partials); index 0 of each kind is the largest
SHAPES = [
    (2, 8, 2, 700, 700, 128, True),
    (1, 8, 2, 300, 260, 128, True),
    (2, 16, 4, 1, 6000, 128, False),
    (1, 16, 4, 4, 2500, 128, False),
    (1, 4, 1, 130, 130, 64, True),
]


def _stats():
    import rdnattention

    return rdnattention.scratch_stats(torch.cuda.current_device())


def test_warm_streams_make_no_allocator_call(gpu):
    """After each of three streams has run the largest call of every kind,
    100 calls of those shapes and smaller ones, spread over the three streams,
    make no allocator call and leave the device's free memory unchanged, and
    every output is bit-identical to the same call on the default stream.
    One growth step afterwards makes exactly one allocator call; the calls
    after it make none."""
    import rdnattention

    streams = [torch.cuda.Stream() for _ in range(3)]
    cases = []
    for i, (b, hq, hkv, sq, sk, d, causal) in enumerate(SHAPES):
        q, k, v, cos, sin = _inputs(gpu, 200 + i, b, hq, hkv, sq, sk, d)
        want = torch.empty_like(q)
        assert forward_raw(q, k, v, want, causal, -1, cos, sin) == 0
        outs = [torch.empty_like(q) for _ in streams]
        cases.append((q, k, v, cos, sin, causal, want, outs))
    torch.cuda.synchronize()
    rdnattention.trim_scratch()
    log("[scratch] warm-up: every shape on every stream")
    for s in streams:
        with torch.cuda.stream(s):
            for q, k, v, cos, sin, causal, _, outs in cases:
                assert forward_raw(q, k, v, outs[0], causal, -1, cos, sin) == 0
    torch.cuda.synchronize()
    warm = _stats()
    free0 = torch.cuda.mem_get_info()[0]
    log(f"[scratch] warm: {warm}; 100 calls over 3 streams")
    for n in range(100):
        si = n % 3
        q, k, v, cos, sin, causal, _, outs = cases[(7 * n + si) % len(cases)]
        with torch.cuda.stream(streams[si]):
            assert forward_raw(q, k, v, outs[si], causal, -1, cos, sin) == 0
    torch.cuda.synchronize()
    assert _stats() == warm
    assert torch.cuda.mem_get_info()[0] == free0
    for q, k, v, cos, sin, causal, want, outs in cases:
        for si in range(3):
            with torch.cuda.stream(streams[si]):
                assert forward_raw(q, k, v, outs[si], causal, -1, cos, sin) == 0
        torch.cuda.synchronize()
        for o in outs:
            assert torch.equal(o.view(torch.int16), want.view(torch.int16))
    # one growth step on stream 1: a RoPE decode whose rotated K (2 x 4 x
    # 20000 x 128 fp16, 39 MiB) outgrows every cached copy (at most 12 MiB);
    # its split-K partials fit the cached ones
    log("[scratch] growth step on stream 1")
    q, k, v, cos, sin = _inputs(gpu, 300, 2, 16, 4, 1, 20000, 128)
    big = torch.empty_like(q)
    with torch.cuda.stream(streams[1]):
        assert forward_raw(q, k, v, big, False, -1, cos, sin) == 0
    torch.cuda.synchronize()
    grown = _stats()
    assert grown["allocations"] == warm["allocations"] + 1, (warm, grown)
    assert grown["entries"] == warm["entries"]
    for n in range(30):
        si = n % 3
        with torch.cuda.stream(streams[si]):
            if si == 1:
                assert forward_raw(q, k, v, big, False, -1, cos, sin) == 0
            qq, kk, vv, cc, ss, causal, _, outs = cases[n % len(cases)]
            assert forward_raw(qq, kk, vv, outs[si], causal, -1, cc, ss) == 0
    torch.cuda.synchronize()
    assert _stats()["allocations"] == grown["allocations"]
    rdnattention.trim_scratch()


def _busy(stream, a, b, n):
    with torch.cuda.stream(stream):
        for _ in range(n):
            torch.mm(a, b)


def test_growth_returns_while_stream_busy(gpu):
    """A call whose scratch must grow returns to the host while the work queued
    before it on its stream is still running: the growth is stream-ordered
    (hipFreeAsync / hipMallocAsync), with no hipFree and no host wait.  Its
    result is the same as the warm call's."""
    import rdnattention

    s = torch.cuda.Stream()
    a = torch.randn(8192, 8192, device=gpu, dtype=torch.float16)
    bm = torch.randn(8192, 8192, device=gpu, dtype=torch.float16)
    small = _inputs(gpu, 310, 1, 8, 2, 200, 200, 128)  # rotated K 0.1 MB: one 2 MiB buffer
    large = _inputs(gpu, 311, 2, 8, 4, 3000, 3000, 128)  # rotated K 6.1 MB: grows it
    want = torch.empty_like(large[0])
    got = torch.empty_like(large[0])
    so = torch.empty_like(small[0])
    torch.cuda.synchronize()
    assert forward_raw(*large[:3], want, True, -1, *large[3:]) == 0
    torch.cuda.synchronize()
    rdnattention.trim_scratch()
    with torch.cuda.stream(s):
        assert forward_raw(*small[:3], so, True, -1, *small[3:]) == 0  # stream warm at the small size
    torch.cuda.synchronize()
    before = _stats()
    _busy(s, a, bm, 40)  # ~30 ms of matrix products queued ahead of the call
    t0 = time.perf_counter()
    with torch.cuda.stream(s):
        rc = forward_raw(*large[:3], got, True, -1, *large[3:])
    host_ms = 1e3 * (time.perf_counter() - t0)
    still_busy = not s.query()
    torch.cuda.synchronize()
    log(f"[scratch] growth call: host {host_ms:.3f} ms, stream still busy: {still_busy}")
    assert rc == 0
    assert _stats()["allocations"] == before["allocations"] + 1
    assert still_busy, "the growth call waited for the stream"
    assert host_ms < 10.0, host_ms
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    rdnattention.trim_scratch()


def test_cap_bounds_cached_bytes_over_streams(gpu):
    """Calls on six streams that each cache a 192 MiB rotated-K buffer: the
    device's cached scratch stays within 1 GiB (least recently used idle
    entries are evicted, stream-ordered), and every result is correct."""
    import rdnattention

    cap = 1 << 30
    # K of 1 x 8 x 98304 x 128 fp16 = 192 MiB: its rotated copy fills one cache entry
    b, hq, hkv, sq, sk, d = 1, 8, 8, 2, 98304, 128
    q, k, v, cos, sin = _inputs(gpu, 320, b, hq, hkv, sq, sk, d)
    want = torch.empty_like(q)
    assert forward_raw(q, k, v, want, False, -1, cos, sin) == 0
    torch.cuda.synchronize()
    rdnattention.trim_scratch()
    streams = [torch.cuda.Stream() for _ in range(6)]
    outs = [torch.empty_like(q) for _ in streams]
    for rep in range(2):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                assert forward_raw(q, k, v, outs[i], False, -1, cos, sin) == 0
            st = _stats()
            log(f"[scratch] rep {rep} stream {i}: {st}")
            assert st["cached_bytes"] <= cap, st
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o.view(torch.int16), want.view(torch.int16))
    rdnattention.trim_scratch()
    assert _stats()["cached_bytes"] == 0
