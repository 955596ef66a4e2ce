"""The library under HIP graph capture (torch.cuda.graph): the FP16 prefill
path with RoPE (K pre-rotation into stream-ordered scratch), the split-K
decode path (partials in scratch, combine kernel) and the quantised INT8 path
(quantiser kernels with scratch, INT8 kernel with the fused channel scales).
Each graph is replayed several times with eager work and synchronisation in
between (the outputs are cleared), and every replay must reproduce the eager
result bit for bit."""
import pytest
import torch

import oracle
from tests.gpu_util import log

pytestmark = pytest.mark.gpu


def _check_replays(fn, outs, n=3):
    torch.cuda.synchronize()
    fn()
    torch.cuda.synchronize()
    ref = [o.clone() for o in outs()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up on the capture stream's side, as torch.cuda.graph expects
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    for rep in range(n):
        for o in outs():
            o.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs(), ref):
            assert torch.equal(o, r), f"replay {rep} differs from the eager result"
    return ref


def test_fp16_rope_prefill_graph(gpu):
    import rdnattention as ra

    log("[graph] fp16 prefill + rope")
    g = torch.Generator().manual_seed(30)
    b, hq, hkv, s, d = 2, 8, 2, 333, 128
    q = torch.randn(b, hq, s, d, generator=g).half().to(gpu)
    k = torch.randn(b, hkv, s, d, generator=g).half().to(gpu)
    v = torch.randn(b, hkv, s, d, generator=g).half().to(gpu)
    cos, sin = (torch.from_numpy(t).to(gpu) for t in oracle.rope_tables(s, d))
    o = torch.empty_like(q)
    ref = _check_replays(lambda: ra.attention_forward_into(q, k, v, o, is_causal=True, rot_cos=cos, rot_sin=sin),
                         lambda: [o])
    assert torch.isfinite(ref[0].float()).all()


def test_splitk_decode_graph(gpu):
    import rdnattention as ra

    log("[graph] split-K decode")
    g = torch.Generator().manual_seed(31)
    b, hq, hkv, sq, sk, d = 2, 8, 2, 1, 4096, 128
    q = torch.randn(b, hq, sq, d, generator=g).half().to(gpu)
    k = torch.randn(b, hkv, sk, d, generator=g).half().to(gpu)
    v = torch.randn(b, hkv, sk, d, generator=g).half().to(gpu)
    o = torch.empty_like(q)
    ref = _check_replays(lambda: ra.attention_forward_into(q, k, v, o, path=ra.PATH_SPLITK), lambda: [o])
    assert torch.isfinite(ref[0].float()).all()


def test_quantized_int8_graph(gpu):
    import rdnattention as ra

    log("[graph] quantised int8 + rope")
    g = torch.Generator().manual_seed(32)
    b, hq, hkv, s, d = 1, 8, 2, 300, 128
    q = torch.randn(b, hq, s, d, generator=g).half().to(gpu)
    k = torch.randn(b, hkv, s, d, generator=g).half().to(gpu)
    v = torch.randn(b, hkv, s, d, generator=g).half().to(gpu)
    cos, sin = (torch.from_numpy(t).to(gpu) for t in oracle.rope_tables(s, d))
    box = {}

    def run():
        box["o"] = ra.flash_attn_int8qk_quantized(q, k, v, is_causal=True, rot_cos=cos, rot_sin=sin)

    # the graph's output is the tensor allocated during capture; eager runs
    # return new tensors, so compare the last eager result with the replays
    torch.cuda.synchronize()
    run()
    torch.cuda.synchronize()
    eager = box["o"].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    out = box["o"]
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from the eager result"
