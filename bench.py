"""Benchmark of the FlashAttention-2 forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
                    [--no-cpu] [--no-secondary]
    python bench.py --copy-calibration          (a plain copy of known size)
    python bench.py --pmc-summary DIR           (rocprofv3 counter CSVs -> table)
    python bench.py --gemm-ceiling 8192         (fp16 torch.matmul: the MFMA ceiling)

Default workload (the headline metric): FP16 causal GQA prefill with
in-kernel RoPE (theta 10000), B=4, Hq=32, Hkv=8, S=key_S=4096, D=128,
Q/K/V ~ N(0,1) fp16 from CPU torch.Generator seed 1, already resident in HBM.
A "step" is one forward over the whole batch through the C ABI (for RoPE
inputs that is the K pre-rotation kernel plus the attention kernel).

Prints ONE JSON line:
  value      TFLOP/s of whole steps (exact masked pair count,
             4*B*Hq*pairs*D FLOPs) over the timed steps, HIP events on
             torch's current stream, which the library launches on; the
             default 50 warmup steps let the GPU clocks reach steady state;
  roofline   the attention kernel alone: FLOPs (or, for decode, algorithmic
             bytes) divided by its mean launch time from the library's kernel
             timer (HIP events recorded around that kernel's launches on its
             stream); `traffic` = HBM bytes per launch from the committed
             rocprofv3 FETCH_SIZE/WRITE_SIZE summary for this kernel and
             workload, scaled by the copy calibration it records, or null;
  cpu_baseline  the CPU oracle (C, fp64, threaded) on a bounded sample of
             the same workload on the host cores ("port");
  cpu_sdpa   torch's CPU scaled_dot_product_attention on a bounded sample;
  parity_vs_oracle  the measured step's output on the CPU baseline's sample
             against the oracle's output there (max/mean abs, rel_rms);
  secondary  the other measured shapes: INT8 vs FP16 on the INT8 shape,
             split-K decode HBM bandwidth, large-head sliding windows.
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import platform
import re
import sys
import time
from dataclasses import dataclass
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP16_PEAK_TFLOPS = 2516.6   # dense fp16 MFMA, 256 CU x 2.4 GHz x 4096 FLOP/clk
INT8_PEAK_TOPS = 5033.2     # dense int8 MFMA
HBM_PEAK_GBS = 8000.0       # HBM3E

METRIC = "attn fwd TFLOPS (fp16) / TOPS (int8), GQA causal S=4096 D=128; % MFMA peak"


@dataclass(frozen=True)
class Workload:
    kind: str        # "f16" (prefill), "int8", "decode" (split-K, strided K/V cache views)
    b: int
    hq: int
    hkv: int
    sq: int
    sk: int
    d: int
    causal: bool
    window: int
    rope: bool
    seed: int
    std: float
    kernel: str      # the main kernel, as rocprofv3 names it
    v_token: bool = False  # int8: V quantised per token, dequantised in the kernel

    @property
    def flops(self) -> int:
        return attn_flops(self.b, self.hq, self.sq, self.sk, self.d, self.causal, self.window)

    @property
    def io_bytes(self) -> int:
        """Algorithmic HBM bytes of one forward: Q, K, V and O once each
        (+ RoPE tables, + per-token scales)."""
        e = 1 if self.kind == "int8" else 2
        n = (self.b * self.hq * self.sq * self.d) * (e + 2) + 2 * self.b * self.hkv * self.sk * self.d * e
        if self.rope:
            n += 2 * max(self.sq, self.sk) * (self.d // 2) * 4
        if self.kind == "int8":
            n += 4 * self.b * (self.hq * self.sq + self.hkv * self.sk)
        if self.v_token:
            n += 4 * self.b * self.hkv * self.sk
        return n


WORKLOADS = {
    "fp16_causal_gqa_rope_b4_h32_kv8_s4096_d128":
        Workload("f16", 4, 32, 8, 4096, 4096, 128, True, -1, True, 1, 1.0, "fa_fwd_f16_pp<128, true>"),
    "fp16_mha_b1_h8_s512_d64":
        Workload("f16", 1, 8, 8, 512, 512, 64, False, -1, False, 0, 1.0, "fa_fwd_f16_pp<64, true>"),
    "int8_causal_gqa_pertoken_b2_h32_kv8_s8192_d128":
        Workload("int8", 2, 32, 8, 8192, 8192, 128, True, -1, False, 3, 1.0, "fa_fwd_int8_f16pv<128, false, false>"),
    "int8_causal_gqa_pertoken_vtoken_b2_h32_kv8_s8192_d128":
        Workload("int8", 2, 32, 8, 8192, 8192, 128, True, -1, False, 3, 1.0, "fa_fwd_int8_f16pv<128, true, false>",
                 True),
    "fp16_causal_gqa_b2_h32_kv8_s8192_d128":
        Workload("f16", 2, 32, 8, 8192, 8192, 128, True, -1, False, 3, 1.0, "fa_fwd_f16_pp<128, true>"),
    # the same shape at head_dim 64, where the INT8 kernel runs both GEMMs on int8 MFMA
    "int8_causal_gqa_pertoken_b2_h32_kv8_s8192_d64":
        Workload("int8", 2, 32, 8, 8192, 8192, 64, True, -1, False, 3, 1.0, "fa_fwd_int8<64, true, false>"),
    "fp16_causal_gqa_b2_h32_kv8_s8192_d64":
        Workload("f16", 2, 32, 8, 8192, 8192, 64, True, -1, False, 3, 1.0, "fa_fwd_f16_pp<64, true>"),
    "fp16_decode_b16_h32_kv8_sq1_sk32768_d128":
        Workload("decode", 16, 32, 8, 1, 32768, 128, False, -1, False, 4, 1.0, "fa_fwd_f16_decode<128>"),
    "fp16_decode_b16_h32_kv8_sq4_sk32768_d128":
        Workload("decode", 16, 32, 8, 4, 32768, 128, False, -1, False, 4, 1.0, "fa_fwd_f16_decode<128>"),
    "fp16_window4096_rope_b1_h16_s16384_d256":
        Workload("f16", 1, 16, 16, 16384, 16384, 256, False, 4096, True, 5, 0.5, "fa_fwd_f16_kpair<256, false>"),
    "fp16_window4096_rope_b1_h16_s4096_d512":
        Workload("f16", 1, 16, 16, 4096, 4096, 512, False, 4096, True, 6, 0.5, "fa_fwd_f16_dpair<512, false>"),
}
DEFAULT = "fp16_causal_gqa_rope_b4_h32_kv8_s4096_d128"
SECONDARY = [
    "int8_causal_gqa_pertoken_b2_h32_kv8_s8192_d128",
    "int8_causal_gqa_pertoken_vtoken_b2_h32_kv8_s8192_d128",
    "fp16_causal_gqa_b2_h32_kv8_s8192_d128",
    "int8_causal_gqa_pertoken_b2_h32_kv8_s8192_d64",
    "fp16_causal_gqa_b2_h32_kv8_s8192_d64",
    "fp16_decode_b16_h32_kv8_sq1_sk32768_d128",
    "fp16_decode_b16_h32_kv8_sq4_sk32768_d128",
    "fp16_window4096_rope_b1_h16_s16384_d256",
    "fp16_window4096_rope_b1_h16_s4096_d512",
]


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
    convention of the reference's tests/benchmark.py:77-88, extended to windows
    (bottom-right aligned, delta = sk - sq; one-sided causal window w keeps
    keys with q+delta-k < w, a two-sided one |q+delta-k| <= w/2)."""
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
    """Interleaved-pair RoPE with torch ops (fp32), for the CPU SDPA baseline."""
    s = x.shape[-2]
    c, sn = cos[:s], sin[:s]
    a, b = x[..., 0::2], x[..., 1::2]
    y = x.clone()
    y[..., 0::2] = a * c - b * sn
    y[..., 1::2] = a * sn + b * c
    return y


# --------------------------------------------------------------------------- #
# inputs and one step per workload kind
# --------------------------------------------------------------------------- #
def cpu_inputs(wl: Workload):
    """The headline's inputs: CPU torch.Generator(seed) N(0, std) -> fp16."""
    import torch

    g = torch.Generator().manual_seed(wl.seed)
    q = (torch.randn(wl.b, wl.hq, wl.sq, wl.d, generator=g) * wl.std).half()
    k = (torch.randn(wl.b, wl.hkv, wl.sk, wl.d, generator=g) * wl.std).half()
    v = (torch.randn(wl.b, wl.hkv, wl.sk, wl.d, generator=g) * wl.std).half()
    cos = sin = None
    if wl.rope:
        cos, sin = rope_tables(max(wl.sq, wl.sk), wl.d)
    return q, k, v, cos, sin


def make_step(wl: Workload, dev, host=None):
    """Device inputs (moved from `host`, or drawn on the GPU from the
    workload's seed) and a closure running one forward."""
    import torch

    import rdnattention as ra

    g = torch.Generator(device=dev).manual_seed(wl.seed)

    def randn(*shape):
        return torch.randn(*shape, device=dev, generator=g) * wl.std

    if wl.kind == "f16":
        if host is not None:
            q, k, v, cos, sin = host
            q, k, v = q.to(dev), k.to(dev), v.to(dev)
        else:
            q = randn(wl.b, wl.hq, wl.sq, wl.d).half()
            k = randn(wl.b, wl.hkv, wl.sk, wl.d).half()
            v = randn(wl.b, wl.hkv, wl.sk, wl.d).half()
            cos = sin = None
            if wl.rope:
                cos, sin = rope_tables(max(wl.sq, wl.sk), wl.d)
        cos = cos.to(dev) if cos is not None else None
        sin = sin.to(dev) if sin is not None else None
        out = torch.empty_like(q)

        def step():
            ra.attention_forward_into(q, k, v, out, is_causal=wl.causal, window_size=wl.window, rot_cos=cos,
                                      rot_sin=sin)

        step.out = out
        return step
    if wl.kind == "int8":
        qf = randn(wl.b, wl.hq, wl.sq, wl.d)
        kf = randn(wl.b, wl.hkv, wl.sk, wl.d)
        vf = randn(wl.b, wl.hkv, wl.sk, wl.d)
        qi, ki, q_scale, k_scale = ra.quantize_int8_qk_pertoken(qf, kf)
        if wl.v_token:
            vi, v_tok = ra.quantize_int8_pertoken_v(vf)
            v_scale = 1.0
        else:
            _, _, vi, _, _, v_scale, _ = ra.quantize_int8_perchannel_v(qf, kf, vf)
            v_tok = None
        del qf, kf, vf
        out = torch.empty(qi.shape, dtype=torch.float16, device=dev)
        return lambda: ra.attention_int8_forward_into(qi, ki, vi, out, q_scale, k_scale, v_scale,
                                                      is_causal=wl.causal, window_size=wl.window, v_token=v_tok)
    if wl.kind == "decode":
        # K/V are views of one [B, S, 2, Hkv, D] cache: head stride D, seq stride 2*Hkv*D
        cache = randn(wl.b, wl.sk, 2, wl.hkv, wl.d).half()
        k = cache[:, :, 0].transpose(1, 2)
        v = cache[:, :, 1].transpose(1, 2)
        q = randn(wl.b, wl.hq, wl.sq, wl.d).half()
        out = torch.empty_like(q)
        return lambda: ra.attention_forward_into(q, k, v, out, is_causal=wl.causal, window_size=wl.window)
    raise ValueError(wl.kind)


def int8_quantized_e2e(dev, steps: int = 10, warmup: int = 20):
    """flash_attn_int8qk_quantized on fp16 inputs of the INT8 workload's shape
    (B=2, Hq=32, Hkv=8, S=8192, D=128, causal), timed whole: this library's
    path (three quantiser kernels + the INT8 kernel with the per-channel V
    rescale in its epilogue) against the reference wrapper's composition
    (rdnattention/__init__.py:303-357: torch quantisers, including the
    per-tensor Q/K pass it discards, the INT8 kernel, then a torch multiply of
    the output by v_channel)."""
    import torch

    import rdnattention as ra

    g = torch.Generator(device=dev).manual_seed(7)
    b, hq, hkv, s, d = 2, 32, 8, 8192, 128
    q = torch.randn(b, hq, s, d, device=dev, generator=g).half()
    k = torch.randn(b, hkv, s, d, device=dev, generator=g).half()
    v = torch.randn(b, hkv, s, d, device=dev, generator=g).half()

    def torch_composition():
        def per_tensor(x):
            sc = x.abs().max().item() / 127.0
            sc = sc if sc != 0.0 else 1.0
            return torch.clamp(torch.round(x / sc), -127, 127).to(torch.int8), sc

        def per_token(x):
            x = x.float()
            sc = x.abs().amax(dim=-1, keepdim=True) / 127.0
            sc = torch.where(sc == 0, torch.ones_like(sc), sc)
            return torch.clamp(torch.round(x / sc), -127, 127).to(torch.int8), sc.squeeze(-1).contiguous()

        per_tensor(q.float())
        per_tensor(k.float())
        vf = v.float()
        vc = vf.abs().amax(dim=-2, keepdim=True) / 127.0
        vc = torch.where(vc == 0, torch.ones_like(vc), vc)
        vi = torch.clamp(torch.round(vf / vc), -127, 127).to(torch.int8)
        qi, qs = per_token(q)
        ki, ks = per_token(k)
        out = ra.flash_attn_int8qk(qi, ki, vi, qs, ks, 1.0, True)
        return (out.float() * vc.repeat_interleave(hq // hkv, dim=1)).to(out.dtype)

    def fused():
        return ra.flash_attn_int8qk_quantized(q, k, v, is_causal=True)

    res = {}
    for name, fn in (("fused_ms", fused), ("torch_composition_ms", torch_composition)):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        res[name] = round((time.perf_counter() - t0) * 1e3 / steps, 4)
    res["speedup"] = round(res["torch_composition_ms"] / res["fused_ms"], 2)
    res["shape"] = "fp16 Q [2,32,8192,128], K/V [2,8,8192,128], causal"
    return res


def time_steps(step, steps: int, warmup: int):
    """Runs `warmup` untimed steps, then `steps` timed ones bracketed by
    device synchronisation (HIP events on torch's stream; no other
    instrumentation), then the same number again under the library's kernel
    timer for the kernels' own time.  Returns (ms per step, mean kernel ms,
    kernel launches, wall s of the timed steps)."""
    import torch

    import rdnattention as ra

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        step()
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start.elapsed_time(stop) / steps
    with ra.KernelTimer() as kt:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    return ms_step, kt.mean_ms, kt.launches, wall


def roofline(wl: Workload, kernel_ms: float, traffic):
    if wl.kind == "decode":
        achieved = wl.io_bytes / (kernel_ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic}
    peak = INT8_PEAK_TOPS if wl.kind == "int8" else FP16_PEAK_TFLOPS
    achieved = wl.flops / (kernel_ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak,
            "unit": "TOP/s" if wl.kind == "int8" else "TFLOP/s", "frac": round(achieved / peak, 4),
            "traffic": traffic}


def profiled_traffic(name: str, wl: Workload):
    """HBM bytes per launch of the workload's main kernel, from the committed
    rocprofv3 counter summary profiles/<kernel>__<workload>.md (its
    "traffic_bytes_per_launch:" line), or None when there is none."""
    kern = re.sub(r"[<>, ]+", "_", wl.kernel).strip("_")
    path = ROOT / "profiles" / f"{kern}__{name}.md"
    try:
        text = path.read_text()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)\s*$", text, re.M)
    return int(m.group(1)) if m else None


# --------------------------------------------------------------------------- #
# CPU baselines
# --------------------------------------------------------------------------- #
def cpu_oracle_baseline(wl: Workload, host, budget_s: float = 12.0):
    """The CPU oracle (oracle/attn_oracle.c: fp64 accumulation, threaded over
    (batch, head, 64-row chunks)) on a bounded sample of the workload: the
    first n (batch, kv head) units in batch-major order with their query
    heads, full sequence, RoPE applied by the oracle first.  FLOPs counted
    like the GPU's."""
    import oracle

    q, k, v, cos, sin = host
    ratio = wl.hq // wl.hkv
    units = wl.b * wl.hkv
    threads = oracle.default_threads()
    # flattening batch into heads keeps the GQA map: (b*Hq + h) / ratio = b*Hkv + h/ratio
    qn = q.float().reshape(1, wl.b * wl.hq, wl.sq, wl.d).numpy()
    kn = k.float().reshape(1, units, wl.sk, wl.d).numpy()
    vn = v.float().reshape(1, units, wl.sk, wl.d).numpy()
    cn = cos.numpy() if cos is not None else None
    sn = sin.numpy() if sin is not None else None

    def run(n):
        qs, ks, vs = qn[:, : n * ratio], kn[:, :n], vn[:, :n]
        t0 = time.perf_counter()
        if wl.rope:
            qs = oracle.rope(qs, cn, sn)
            ks = oracle.rope(ks, cn, sn)
        o = oracle.attention(qs, ks, vs, causal=wl.causal, window=wl.window, nthreads=threads)
        return time.perf_counter() - t0, o

    t1, _ = run(1)
    n = max(1, min(units, int(budget_s / max(t1, 1e-6))))
    t, ref = run(n)
    flops = attn_flops(1, n * ratio, wl.sq, wl.sk, wl.d, wl.causal, wl.window)
    return {"value": round(flops / t / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": (f"CPU oracle (C, fp64 accumulation, {threads} threads) on {cpu_model()} "
                       f"(os.cpu_count()={os.cpu_count()}): {n} of {units} (batch, kv head) units = "
                       f"{n * ratio} of {wl.b * wl.hq} query-head rows of S={wl.sq}, RoPE included, "
                       f"one run of {t:.2f} s")}, ref


def sample_parity(wl: Workload, gpu_out, ref):
    """The GPU output of the measured step against the oracle's output for the
    CPU baseline's sample (its first query heads in batch-major order): max
    and mean absolute error and rel_rms, with the FP16 bars they must meet."""
    import numpy as np

    rows = ref.shape[1]
    got = gpu_out.reshape(1, wl.b * wl.hq, wl.sq, wl.d)[:, :rows].float().cpu().numpy().astype(np.float64)
    d = np.abs(got - ref)
    rr = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
    res = {"max_abs": float(d.max()), "mean_abs": float(d.mean()),
           "rel_rms": float(np.sqrt((d ** 2).mean()) / rr) if rr > 0 else float(np.sqrt((d ** 2).mean())),
           "query_head_rows": f"{rows} of {wl.b * wl.hq}", "bar": {"max_abs": 2e-3, "mean_abs": 2e-4}}
    res["ok"] = bool(np.isfinite(got).all() and res["max_abs"] <= 2e-3 and res["mean_abs"] <= 2e-4)
    return res


def cpu_sdpa_baseline(wl: Workload, host, budget_s: float = 12.0):
    """torch CPU scaled_dot_product_attention (fp32, torch's default threads)
    on a bounded sample: the first n (batch, kv head) units, full S."""
    import torch

    q, k, v, cos, sin = host
    ratio = wl.hq // wl.hkv
    units = wl.b * wl.hkv
    delta = wl.sk - wl.sq
    qf = q.reshape(1, wl.b * wl.hq, wl.sq, wl.d)
    kf = k.reshape(1, units, wl.sk, wl.d)
    vf = v.reshape(1, units, wl.sk, wl.d)

    def run(n):
        qs = qf[:, : n * ratio].float()
        ks = kf[:, :n].float()
        vs = vf[:, :n].float()
        t0 = time.perf_counter()
        if wl.rope:
            qs = rope_interleaved(qs, cos, sin)
            ks = rope_interleaved(ks, cos, sin)
        mask = None
        is_causal = False
        if wl.window > 0 or (wl.causal and delta != 0):
            i = torch.arange(wl.sq)[:, None] + delta
            j = torch.arange(wl.sk)[None, :]
            mask = torch.ones(wl.sq, wl.sk, dtype=torch.bool)
            if wl.causal:
                mask &= j <= i
            if wl.window > 0:
                mask &= (i - j < wl.window) if wl.causal else ((i - j).abs() <= wl.window // 2)
        elif wl.causal:
            is_causal = True
        torch.nn.functional.scaled_dot_product_attention(qs, ks, vs, attn_mask=mask, is_causal=is_causal,
                                                         enable_gqa=ratio > 1)
        return time.perf_counter() - t0

    run(1)
    t1 = run(1)
    n = max(1, min(units, int(budget_s / 3 / max(t1, 1e-6))))
    t = sorted(run(n) for _ in range(3))[1]
    flops = attn_flops(1, n * ratio, wl.sq, wl.sk, wl.d, wl.causal, wl.window)
    return {"value": round(flops / t / 1e12, 5), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "torch",
            "sample": (f"torch.nn.functional.scaled_dot_product_attention fp32 on {cpu_model()}: {n} of {units} "
                       f"(batch, kv head) units = {n * ratio} of {wl.b * wl.hq} query-head rows of S={wl.sq}, "
                       f"RoPE with torch ops included, median of 3 runs ({t:.2f} s)")}


# --------------------------------------------------------------------------- #
# profiling helpers (run under rocprofv3 / on its output)
# --------------------------------------------------------------------------- #
COPY_BYTES = 1 << 30


def copy_calibration(steps: int = 5) -> int:
    """A plain device-to-device copy of COPY_BYTES (1 GiB read, 1 GiB written)
    per launch, `steps` launches: under rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    its per-dispatch KiB give the counters' scale against known traffic."""
    import torch

    src = torch.ones(COPY_BYTES // 2, dtype=torch.float16, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": COPY_BYTES, "launches": steps}), flush=True)
    return 0


def gemm_ceiling(n: int = 8192, steps: int = 20, warmup: int = 50) -> int:
    """The practical fp16 MFMA ceiling of this GPU: torch.matmul (hipBLASLt)
    of two n x n fp16 matrices, timed with HIP events after `warmup` untimed
    products (the clock ramp), 2 n^3 FLOPs each.  Run it under rocprofv3
    --pmc SQ_VALU_MFMA_BUSY_CYCLES ... for the library GEMM's MFMA-busy share."""
    import torch

    g = torch.Generator(device="cuda:0").manual_seed(0)
    a = torch.randn(n, n, device="cuda:0", generator=g).half()
    b = torch.randn(n, n, device="cuda:0", generator=g).half()
    for _ in range(warmup):
        c = torch.matmul(a, b)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        c = torch.matmul(a, b)
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    tflops = 2 * n ** 3 / (ms * 1e-3) / 1e12
    print(json.dumps({"gemm": f"fp16 {n}x{n}x{n} torch.matmul", "ms": round(ms, 4), "tflops": round(tflops, 1),
                      "frac_of_dense_peak": round(tflops / FP16_PEAK_TFLOPS, 4), "checksum": float(c[0, 0])}),
          flush=True)
    return 0


def pmc_summary(directory: str) -> int:
    """Mean per-dispatch counter values per kernel from rocprofv3's
    *counter_collection.csv files under `directory`."""
    acc = {}
    for path in sorted(Path(directory).rglob("*counter_collection.csv")):
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                key = (row["Kernel_Name"], row["Counter_Name"])
                s, n = acc.get(key, (0.0, 0))
                acc[key] = (s + float(row["Counter_Value"]), n + 1)
    if not acc:
        print(f"no counter_collection.csv under {directory}", file=sys.stderr)
        return 1
    for (kern, ctr), (s, n) in sorted(acc.items()):
        print(f"{ctr:<28} dispatches={n:<5} mean={s / n:16.1f}  {kern[:110]}")
    for line in pmc_derived(directory, {k: s / n for k, (s, n) in acc.items()}):
        print(line)
    return 0


def trace_steps(directory: str, main: str, last: int = 40) -> int:
    """Per-step timeline of the last `last` steps from rocprofv3's
    *kernel_trace.csv under `directory`.  A step ends with a dispatch whose
    kernel name contains `main` and holds every dispatch since the previous
    one: its time is end-to-end between the two main dispatches' ends, split
    into each kernel's own time and the gaps between dispatches (launch and
    completion latency, queue packets)."""
    rows = []
    for path in sorted(Path(directory).rglob("*kernel_trace.csv")):
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                rows.append((int(row["Start_Timestamp"]), int(row["End_Timestamp"]), row["Kernel_Name"]))
    rows.sort()
    ends = [i for i, r in enumerate(rows) if main in r[2]]
    if len(ends) < 2:
        print(f"fewer than two '{main}' dispatches under {directory}", file=sys.stderr)
        return 1
    ends = ends[-(last + 1):]
    per_kernel, gaps, steps = {}, [], []
    for a, b in zip(ends, ends[1:]):
        step = rows[b][1] - rows[a][1]
        busy = 0
        for r in rows[a + 1:b + 1]:
            name = r[2].replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0][:60]
            per_kernel.setdefault(name, []).append(r[1] - r[0])
            busy += r[1] - r[0]
        steps.append(step)
        gaps.append(step - busy)
    n = len(steps)
    print(f"steps={n} mean_step_us={sum(steps) / n / 1e3:.2f} gaps_us={sum(gaps) / n / 1e3:.2f}")
    for name, d in per_kernel.items():
        print(f"  {name:<62} per_step_us={sum(d) / n / 1e3:9.2f} calls_per_step={len(d) / n:.0f}")
    return 0


def pmc_derived(directory: str, mean):
    """Derived per-kernel figures from mean per-dispatch counters (and, when
    a run_kernel_trace.csv is present, mean dispatch durations):
      mfma_busy  SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x SIMDs):
                 the share of SIMD cycles the matrix core is busy at the clock
                 it ran at (the busy-cycle counter is 32 cycles per 32x32x16
                 f16 or 32x32x32 i8 MFMA issued; GRBM_GUI_ACTIVE is summed
                 over the XCDs);
      sclk       GRBM_GUI_ACTIVE / XCDs cycles / mean duration;
      valu/mfma  non-MFMA VALU instructions per MFMA instruction;
      lds_conflict_per_inst  SQ_LDS_BANK_CONFLICT cycles per LDS instruction;
      lds_util   SQ_LDS_IDX_ACTIVE / (GRBM_GUI_ACTIVE / XCDs x CUs): the share
                 of cycles each CU's LDS is busy with indexed (ds_*) accesses
                 (rocprofv3's LdsUtil);
      wait       SQ_WAIT_ANY / SQ_WAVE_CYCLES: the share of wave time spent
                 waiting (on memory, LDS, barriers or dependencies)."""
    simds, xcds, cus = 1024, 8, 256
    for path in Path(directory).rglob("*agent_info.csv"):
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                if row.get("Agent_Type") == "GPU" and int(row.get("Simd_Count", 0) or 0) > 0:
                    simds = int(row["Simd_Count"])
                    xcds = max(1, int(row.get("Num_Xcc", 1) or 1))
                    cus = int(row.get("Cu_Count", cus) or cus)
    dur = {}
    for path in Path(directory).rglob("*kernel_trace.csv"):
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                s, n = dur.get(row["Kernel_Name"], (0.0, 0))
                dur[row["Kernel_Name"]] = (s + int(row["End_Timestamp"]) - int(row["Start_Timestamp"]), n + 1)
    out = []
    for kern in sorted({k for k, _ in mean}):
        def c(name):
            return mean.get((kern, name))

        items = []
        busy, gui = c("SQ_VALU_MFMA_BUSY_CYCLES"), c("GRBM_GUI_ACTIVE")
        gui = gui / xcds if gui else gui
        if busy is not None and gui:
            items.append(f"mfma_busy={busy / (gui * simds):.4f}")
        if gui and kern in dur:
            ns = dur[kern][0] / dur[kern][1]
            items.append(f"sclk_mhz={gui / ns * 1e3:.0f}")
        valu, mfma = c("SQ_INSTS_VALU"), c("SQ_INSTS_MFMA")
        if valu is not None and mfma:
            items.append(f"valu_non_mfma_per_mfma={(valu - mfma) / mfma:.2f}")
        trans = c("SQ_INSTS_VALU_TRANS_F32")
        if trans is not None and mfma:
            items.append(f"trans_per_mfma={trans / mfma:.3f}")
        conf, lds = c("SQ_LDS_BANK_CONFLICT"), c("SQ_INSTS_LDS")
        if conf is not None and lds:
            items.append(f"lds_conflict_cycles_per_inst={conf / lds:.4f}")
        idx = c("SQ_LDS_IDX_ACTIVE")
        if idx is not None and gui:
            items.append(f"lds_util={idx / (gui * cus):.4f}")
        wait, wave_cycles = c("SQ_WAIT_ANY"), c("SQ_WAVE_CYCLES")
        if wait is not None and wave_cycles:
            items.append(f"wait={wait / wave_cycles:.4f}")
        if items:
            out.append(f"derived {kern[:90]}: " + " ".join(items))
    return out


# --------------------------------------------------------------------------- #
def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # GPU clocks ramp up over the first ~20 ms of sustained load: 50 untimed
    # steps (~35 ms at the default workload) put the timed steps at steady state
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default=DEFAULT, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--no-secondary", action="store_true", help="measure the selected workload only")
    ap.add_argument("--copy-calibration", action="store_true", help="run the 1 GiB copy used to scale counters")
    ap.add_argument("--pmc-summary", metavar="DIR", help="summarise rocprofv3 counter CSVs under DIR")
    ap.add_argument("--trace-steps", nargs=2, metavar=("DIR", "KERNEL"),
                    help="per-step kernel times and dispatch gaps of the last 40 steps ending with KERNEL, "
                         "from rocprofv3 kernel-trace CSVs under DIR")
    ap.add_argument("--gemm-ceiling", type=int, metavar="N", default=0,
                    help="time an N^3 fp16 torch.matmul (the practical MFMA ceiling) and exit")
    args = ap.parse_args(argv)
    if args.pmc_summary:
        return pmc_summary(args.pmc_summary)
    if args.trace_steps:
        return trace_steps(args.trace_steps[0], args.trace_steps[1])
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(attention shards by (batch, kv head) with no exchange); run with --gpus 1", file=sys.stderr)
        return 2
    if args.copy_calibration:
        return copy_calibration()
    if args.gemm_ceiling:
        return gemm_ceiling(args.gemm_ceiling)

    import torch

    import rdnattention as ra

    dev = torch.device("cuda:0")
    name = args.workload
    wl = WORKLOADS[name]
    host = cpu_inputs(wl) if wl.kind == "f16" else None
    step = make_step(wl, dev, host)
    # The secondary workloads are measured after the headline's inputs are
    # built (host-only work, during which the clocks fall back) and right
    # before its timing: the headline's warmup and timed steps then run at the
    # clocks that sustained load holds (they ramp over the first ~20 ms, longer
    # than a few warmup steps of the headline).
    secondary = {}
    if not args.no_secondary and name == DEFAULT:
        # the end-to-end INT8 comparison first: its torch-op composition
        # leaves the GPU partly idle, and the clocks drop with it
        try:
            secondary["int8_quantized_end_to_end"] = int8_quantized_e2e(dev)
        except ra.RDNAttentionError as e:
            secondary["int8_quantized_end_to_end"] = {"error": str(e)}
        torch.cuda.empty_cache()
        for other in SECONDARY:
            owl = WORKLOADS[other]
            try:
                ostep = make_step(owl, dev)
                oms, okms, _, _ = time_steps(ostep, 10, 20)
                del ostep
                rf = roofline(owl, okms, profiled_traffic(other, owl))
                secondary[other] = {"ms_per_step": round(oms, 4), "kernel_ms": round(okms, 4), "roofline": rf}
            except ra.RDNAttentionError as e:
                secondary[other] = {"error": str(e)}
            torch.cuda.empty_cache()
        i8 = secondary.get("int8_causal_gqa_pertoken_b2_h32_kv8_s8192_d128", {})
        f16 = secondary.get("fp16_causal_gqa_b2_h32_kv8_s8192_d128", {})
        if "kernel_ms" in i8 and "kernel_ms" in f16:
            secondary["int8_over_fp16_same_shape"] = round(f16["kernel_ms"] / i8["kernel_ms"], 3)
        i8d64 = secondary.get("int8_causal_gqa_pertoken_b2_h32_kv8_s8192_d64", {})
        f16d64 = secondary.get("fp16_causal_gqa_b2_h32_kv8_s8192_d64", {})
        if "kernel_ms" in i8d64 and "kernel_ms" in f16d64:
            secondary["int8_over_fp16_same_shape_d64"] = round(f16d64["kernel_ms"] / i8d64["kernel_ms"], 3)
        i8t = secondary.get("int8_causal_gqa_pertoken_vtoken_b2_h32_kv8_s8192_d128", {})
        if "kernel_ms" in i8 and "kernel_ms" in i8t:
            secondary["int8_vtoken_time_over_int8"] = round(i8t["kernel_ms"] / i8["kernel_ms"], 3)

    ms_step, kernel_ms, launches, wall = time_steps(step, args.steps, args.warmup)
    if launches != args.steps:
        raise RuntimeError(f"kernel timer saw {launches} launches for {args.steps} steps")
    if wl.kind == "decode":
        value, unit = wl.io_bytes / (ms_step * 1e-3) / 1e9, "GB/s"
    else:
        value, unit = wl.flops / (ms_step * 1e-3) / 1e12, ("TOP/s" if wl.kind == "int8" else "TFLOP/s")

    cpu = sdpa = parity = None
    if not args.no_cpu and host is not None:
        cpu, ref = cpu_oracle_baseline(wl, host)
        parity = sample_parity(wl, step.out, ref)
        del ref
        sdpa = cpu_sdpa_baseline(wl, host)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"f16": "fp16", "int8": "int8", "decode": "fp16"}[wl.kind],
        "data": ("synthetic N(0,%g) from torch.Generator(seed=%d), resident in HBM" % (wl.std, wl.seed)),
        "config": {"workload": name, "batch": wl.b, "num_heads": wl.hq, "num_kv_heads": wl.hkv,
                   "seq_len": wl.sq, "key_seq_len": wl.sk, "head_dim": wl.d, "causal": wl.causal,
                   "window_size": wl.window, "rope": wl.rope, "parallelism": "single GPU"},
        "roofline": roofline(wl, kernel_ms, profiled_traffic(name, wl)),
        "cpu_baseline": cpu,
        "cpu_sdpa": sdpa,
        "parity_vs_oracle": parity,
        "kernel": wl.kernel,
        "kernel_ms_mean": round(kernel_ms, 4),
        "algorithmic_bytes_per_launch": wl.io_bytes,
        "secondary": secondary or None,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
