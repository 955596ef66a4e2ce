"""Benchmark of the FlashAttention-2 forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Default workload (the headline metric): FP16 causal GQA prefill with
in-kernel RoPE (theta 10000), B=4, Hq=32, Hkv=8, S=key_S=4096, D=128,
Q/K/V ~ N(0,1) fp16 from CPU torch.Generator seed 1, already resident in HBM.
A "step" is one forward over the whole batch through the C ABI.

Prints ONE JSON line: value = TFLOP/s over the timed steps (exact masked
pair count, 4*B*Hq*pairs*D FLOPs), roofline of the attention kernel from
HIP events on its stream, and a CPU baseline (torch SDPA on host cores on a
bounded sample of the same workload).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP16_PEAK_TFLOPS = 2516.6   # dense fp16 MFMA, 256 CU x 2.4 GHz x 4096 FLOP/clk
INT8_PEAK_TOPS = 5033.2     # dense int8 MFMA
HBM_PEAK_GBS = 8000.0       # HBM3E

METRIC = "attn fwd TFLOPS (fp16) / TOPS (int8), GQA causal S=4096 D=128; % MFMA peak"

WORKLOADS = {
    # name: (B, Hq, Hkv, Sq, Sk, D, causal, window, rope, seed, std)
    "fp16_causal_gqa_rope_b4_h32_kv8_s4096_d128": (4, 32, 8, 4096, 4096, 128, True, -1, True, 1, 1.0),
    "fp16_mha_b1_h8_s512_d64": (1, 8, 8, 512, 512, 64, False, -1, False, 0, 1.0),
    "fp16_window4096_rope_b1_h16_s16384_d256": (1, 16, 16, 16384, 16384, 256, False, 4096, True, 4, 0.5),
    "fp16_window4096_rope_b1_h16_s4096_d512": (1, 16, 16, 4096, 4096, 512, False, 4096, True, 5, 0.5),
}
DEFAULT = "fp16_causal_gqa_rope_b4_h32_kv8_s4096_d128"


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def valid_pairs(sq: int, sk: int, causal: bool, window: int) -> int:
    """Exact number of visible (query, key) pairs of one head: the FLOP-count
    convention of the reference's tests/benchmark.py:77-88, extended to windows."""
    import numpy as np

    i = np.arange(sq, dtype=np.int64) + (sk - sq)
    lo = np.zeros(sq, dtype=np.int64)
    hi = np.full(sq, sk - 1, dtype=np.int64)
    if causal:
        hi = np.minimum(hi, i)
    if window > 0:
        if causal:
            lo = np.maximum(lo, i - window + 1)
        else:
            lo = np.maximum(lo, i - window // 2)
            hi = np.minimum(hi, i + window // 2)
    return int(np.clip(hi - lo + 1, 0, None).sum())


def attn_flops(b, hq, sq, sk, d, causal, window) -> int:
    return 4 * b * hq * valid_pairs(sq, sk, causal, window) * d


def rope_tables(rows: int, head_dim: int, theta: float = 10000.0):
    """fp32 cos/sin [rows, head_dim/2]: ang = pos * theta^(-2i/D) (docs/api.md:84-87)."""
    import torch

    pos = torch.arange(rows, dtype=torch.float32)[:, None]
    inv = theta ** (-torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim)
    ang = pos * inv
    return ang.cos().contiguous(), ang.sin().contiguous()


def rope_interleaved(x, cos, sin):
    """Interleaved-pair RoPE with torch ops (fp32), for the CPU baseline."""
    s = x.shape[-2]
    c, sn = cos[:s], sin[:s]
    a, b = x[..., 0::2], x[..., 1::2]
    y = x.clone()
    y[..., 0::2] = a * c - b * sn
    y[..., 1::2] = a * sn + b * c
    return y


def make_inputs(spec):
    import torch

    b, hq, hkv, sq, sk, d, causal, window, rope, seed, std = spec
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(b, hq, sq, d, generator=g) * std).half()
    k = (torch.randn(b, hkv, sk, d, generator=g) * std).half()
    v = (torch.randn(b, hkv, sk, d, generator=g) * std).half()
    cos = sin = None
    if rope:
        cos, sin = rope_tables(max(sq, sk), d)
    return q, k, v, cos, sin


def cpu_baseline(spec, q, k, v, cos, sin, budget_s=20.0):
    """torch CPU SDPA (fp32) on host cores, on a bounded sample of the workload:
    one batch element and the query heads of as many kv heads as fit the time
    budget, full sequence length.  FLOPs counted like the GPU's."""
    import torch

    b, hq, hkv, sq, sk, d, causal, window, rope, seed, std = spec
    ratio = hq // hkv
    delta = sk - sq

    def run(n_kv):
        qs = q[:1, : n_kv * ratio].float()
        ks = k[:1, :n_kv].float()
        vs = v[:1, :n_kv].float()
        if rope:
            qs = rope_interleaved(qs, cos, sin)
            ks = rope_interleaved(ks, cos, sin)
        mask = None
        is_causal = False
        if window > 0 or (causal and delta != 0):
            i = torch.arange(sq)[:, None] + delta
            j = torch.arange(sk)[None, :]
            mask = torch.ones(sq, sk, dtype=torch.bool)
            if causal:
                mask &= j <= i
            if window > 0:
                mask &= (i - j < window) if causal else ((i - j).abs() <= window // 2)
        elif causal:
            is_causal = True
        t0 = time.perf_counter()
        torch.nn.functional.scaled_dot_product_attention(qs, ks, vs, attn_mask=mask, is_causal=is_causal,
                                                         enable_gqa=ratio > 1)
        return time.perf_counter() - t0

    run(1)  # warm-up (also sizes the sample)
    t1 = min(run(1) for _ in range(2))
    n_kv = max(1, min(hkv, int(budget_s / 3 / max(t1, 1e-6))))
    times = sorted(run(n_kv) for _ in range(3))
    t = times[1]
    flops = attn_flops(1, n_kv * ratio, sq, sk, d, causal, window)
    return {"value": round(flops / t / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"torch.nn.functional.scaled_dot_product_attention fp32 on the host CPU "
                       f"({cpu_model()}, os.cpu_count()={os.cpu_count()}), batch 1 of {b}, {n_kv * ratio} of {hq} "
                       f"query heads, full S={sq}, median of 3 runs ({t:.2f} s); the reference has no CPU "
                       f"attention path, so this is the CPU baseline its survey names")}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default=DEFAULT, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(attention shards by (batch, kv head) with no exchange); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    import rdnattention_amd

    spec = WORKLOADS[args.workload]
    b, hq, hkv, sq, sk, d, causal, window, rope, seed, std = spec
    dev = torch.device("cuda:0")
    q, k, v, cos, sin = make_inputs(spec)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    cd = cos.to(dev) if cos is not None else None
    sd = sin.to(dev) if sin is not None else None
    out = torch.empty_like(qd)
    flops = attn_flops(b, hq, sq, sk, d, causal, window)

    def step():
        rdnattention_amd.attention_forward_into(qd, kd, vd, out, is_causal=causal, window_size=window, rot_cos=cd,
                                                rot_sin=sd)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    t0 = time.perf_counter()
    ev[0].record(stream)
    for i in range(args.steps):
        step()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_launch_ms = [ev[i].elapsed_time(ev[i + 1]) for i in range(args.steps)]
    ms_total = ev[0].elapsed_time(ev[-1])
    ms_step = ms_total / args.steps
    tflops = flops / (ms_step * 1e-3) / 1e12
    per_launch_ms.sort()
    med_ms = per_launch_ms[len(per_launch_ms) // 2]
    achieved = flops / (sum(per_launch_ms) / len(per_launch_ms) * 1e-3) / 1e12

    cpu = None if args.no_cpu else cpu_baseline(spec, q, k, v, cos, sin)
    line = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic N(0,1) fp16 from CPU torch.Generator(seed), resident in HBM",
        "config": {"workload": args.workload, "batch": b, "num_heads": hq, "num_kv_heads": hkv, "seq_len": sq,
                   "key_seq_len": sk, "head_dim": d, "causal": causal, "window_size": window, "rope": rope,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / FP16_PEAK_TFLOPS, 4), "traffic": None},
        "cpu_baseline": cpu,
        "kernel_ms_median": round(med_ms, 4),
        "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
