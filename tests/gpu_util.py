"""Helpers shared by the GPU parity tests: input generation, raw C-ABI calls
(strided tensors, forced kernel paths), and the parity bars."""
from __future__ import annotations

import ctypes
import sys

import numpy as np

import oracle

# Parity bars for the FP16 path (max-abs / mean-abs against the CPU reference
# on the same inputs), and the reference gate's own rel_rms bar
# (tests/hip_forward_gate.hip:244).
F16_MAX_ABS = 2e-3
F16_MEAN_ABS = 2e-4
F16_REL_RMS = 5e-3
# INT8: output max-abs against the kernel-exact CPU emulation.
I8_MAX_ABS = 1e-2


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def lib():
    import rdnattention

    return rdnattention._lib_handle()


def stream_ptr():
    import torch

    return torch.cuda.current_stream().cuda_stream


def forward_raw(q, k, v, out, causal=False, window=-1, cos=None, sin=None, scale=None, path=0):
    """rdna_attention_forward_path on (possibly strided) torch tensors."""
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    if scale is None:
        scale = d ** -0.5
    qs, ks, vs, os_ = q.stride(), k.stride(), v.stride(), out.stride()
    rc = lib().rdna_attention_forward_path(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
        cos.data_ptr() if cos is not None else None, sin.data_ptr() if sin is not None else None,
        qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os_[0], os_[1], os_[2],
        b, hq, hkv, sq, sk, d, float(scale), 1 if causal else 0, 1 if cos is not None else 0, int(window),
        int(path), stream_ptr())
    return rc


def seeded_inputs(seed, b, hq, hkv, sq, sk, d, std=1.0):
    """CPU torch.Generator(seed) -> fp32 -> fp16 (the inputs of the measured workloads)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(b, hq, sq, d, generator=g) * std).half()
    k = (torch.randn(b, hkv, sk, d, generator=g) * std).half()
    v = (torch.randn(b, hkv, sk, d, generator=g) * std).half()
    return q, k, v


def lcg_inputs(seed, b, hq, hkv, sq, sk, d, mode=0):
    """The reference gates' inputs: one LCG stream filling Q, then K, then V."""
    import torch

    g = oracle.Lcg(seed)
    q = torch.from_numpy(g.fill((b, hq, sq, d), mode)).half()
    k = torch.from_numpy(g.fill((b, hkv, sk, d), mode)).half()
    v = torch.from_numpy(g.fill((b, hkv, sk, d), mode)).half()
    return q, k, v


def gate_rope_tables(rows, d):
    """tests/hip_forward_gate.hip:150-162: theta = s / 10000^(2p/D) in fp32."""
    half = d // 2
    s = np.arange(rows, dtype=np.float32)[:, None]
    p = np.arange(half, dtype=np.float32)[None, :]
    theta = (s / np.power(np.float32(10000.0), (np.float32(2.0) * p) / np.float32(d))).astype(np.float32)
    return np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)


def reference_f16(q, k, v, causal, window, cos=None, sin=None, scale=None):
    """CPU oracle on the same fp16 inputs; RoPE rotated in fp32 and rounded to
    fp16 like the kernel (src/rdna/fa2_forward_f16.hip:63-77)."""
    qf = q.float().numpy()
    kf = k.float().numpy()
    vf = v.float().numpy()
    if cos is not None:
        qf = oracle.rope(qf, cos, sin, round_f16=True)
        kf = oracle.rope(kf, cos, sin, round_f16=True)
    return oracle.attention(qf, kf, vf, causal=causal, window=window, scale=scale)


def errors(got, ref):
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    d = np.abs(g - r)
    rr = np.sqrt((r ** 2).mean())
    rel = np.sqrt((d ** 2).mean()) / rr if rr > 0 else np.sqrt((d ** 2).mean())
    return float(d.max()), float(d.mean()), float(rel)


def assert_f16_parity(got, ref, name=""):
    mx, mean, rel = errors(got, ref)
    assert np.isfinite(np.asarray(got, dtype=np.float64)).all(), f"{name}: non-finite output"
    assert mx <= F16_MAX_ABS and mean <= F16_MEAN_ABS and rel < F16_REL_RMS, (
        f"{name}: max_abs={mx:.3e} mean_abs={mean:.3e} rel_rms={rel:.3e}")
    return mx, mean, rel
