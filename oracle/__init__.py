"""CPU oracle for the FlashAttention-2 forward path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
import this package, and only to check results against.  The shipped library
(``rdnattention``) never imports it and has no CPU fallback.

This module is a thin numpy/ctypes layer over ``attn_oracle.c`` (built by
``oracle/Makefile`` into ``oracle/liboracle.so``).  The C file restates the
reference's semantics; each function there cites the reference file:line it
follows.  Pinning of every function is in ``tests/test_oracle.py``.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i8p = ctypes.POINTER(ctypes.c_int8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i64 = ctypes.c_int64


def build() -> None:
    """Compile liboracle.so (gcc)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(str(LIB_PATH))
        L.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        L.oracle_half_to_float.restype = ctypes.c_float
        L.oracle_float_to_half.argtypes = [ctypes.c_float]
        L.oracle_float_to_half.restype = ctypes.c_uint16
        L.oracle_visible.argtypes = [_i64, _i64, _i64, _i64, ctypes.c_int32, ctypes.c_int32]
        L.oracle_visible.restype = ctypes.c_int32
        L.oracle_valid_pairs.argtypes = [_i64, _i64, ctypes.c_int32, ctypes.c_int32]
        L.oracle_valid_pairs.restype = _i64
        L.oracle_rope.argtypes = [_f32p, _i64, _i64, _i64, _f32p, _f32p, ctypes.c_int32]
        L.oracle_rope.restype = None
        L.oracle_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64, _i64,
                                       ctypes.c_double, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
        L.oracle_attention.restype = ctypes.c_int32
        L.oracle_int8_scores.argtypes = [_i8p, _i8p, _i32p, _i64, _i64, _i64, _i64, _i64, _i64]
        L.oracle_int8_scores.restype = ctypes.c_int32
        L.oracle_attention_int8.argtypes = [_i8p, _i8p, _i8p, _f32p, _f32p, ctypes.c_float, ctypes.c_float,
                                            ctypes.c_float, _f32p, _i64, _i64, _i64, _i64, _i64, _i64,
                                            ctypes.c_float, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                            ctypes.c_int32]
        L.oracle_attention_int8.restype = ctypes.c_int32
        L.oracle_attention_int8_vtoken.argtypes = [_i8p, _i8p, _i8p, _f32p, _f32p, _f32p, ctypes.c_float,
                                                   ctypes.c_float, ctypes.c_float, _f32p, _i64, _i64, _i64, _i64,
                                                   _i64, _i64, ctypes.c_float, ctypes.c_int32, ctypes.c_int32,
                                                   ctypes.c_int32, ctypes.c_int32]
        L.oracle_attention_int8_vtoken.restype = ctypes.c_int32
        L.oracle_attention_int8_gate.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64, _i64,
                                                 ctypes.c_double, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
        L.oracle_attention_int8_gate.restype = ctypes.c_int32
        L.oracle_quant_pertoken.argtypes = [_f32p, _i64, _i64, _i8p, _f32p]
        L.oracle_quant_pertoken.restype = None
        L.oracle_quant_perchannel.argtypes = [_f32p, _i64, _i64, _i64, _i8p, _f32p]
        L.oracle_quant_perchannel.restype = None
        L.oracle_quant_pertensor.argtypes = [_f32p, _i64, _i8p]
        L.oracle_quant_pertensor.restype = ctypes.c_float
        L.oracle_lcg_fill.argtypes = [_f32p, _i64, _u32p, ctypes.c_int32]
        L.oracle_lcg_fill.restype = None
        _lib = L
    return _lib


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a: np.ndarray, ptype):
    return a.ctypes.data_as(ptype)


# --------------------------------------------------------------------------- #
# fp16 helpers
# --------------------------------------------------------------------------- #
def half_to_float(bits: int) -> float:
    return float(lib().oracle_half_to_float(bits))


def float_to_half(x: float) -> int:
    return int(lib().oracle_float_to_half(x))


def round_f16(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 (RNE) -> fp32 through the oracle's own conversion."""
    x = _c(x, np.float32)
    f = np.vectorize(lambda v: lib().oracle_half_to_float(lib().oracle_float_to_half(float(v))), otypes=[np.float32])
    return f(x).astype(np.float32) if x.size else x


# --------------------------------------------------------------------------- #
# masking / work counting
# --------------------------------------------------------------------------- #
def visible(i: int, k: int, sq: int, sk: int, causal: bool, window: int) -> bool:
    return bool(lib().oracle_visible(i, k, sq, sk, 1 if causal else 0, window))


def valid_pairs(sq: int, sk: int, causal: bool, window: int) -> int:
    return int(lib().oracle_valid_pairs(sq, sk, 1 if causal else 0, window))


def attn_flops(b: int, hq: int, sq: int, sk: int, d: int, causal: bool, window: int) -> int:
    """4 * B * Hq * valid_pairs * D (tests/benchmark.py:77-88 convention)."""
    return 4 * b * hq * valid_pairs(sq, sk, causal, window) * d


# --------------------------------------------------------------------------- #
# RoPE
# --------------------------------------------------------------------------- #
def rope_tables(rows: int, head_dim: int, theta: float = 10000.0):
    """cos/sin tables [rows, head_dim/2] fp32, built the way tests/rope.py:78-81
    and docs/api.md:84-87 build them (fp32: inv = theta^(-2i/D), ang = pos*inv)."""
    pos = np.arange(rows, dtype=np.float32)[:, None]
    inv = (np.float32(theta) ** (-(np.arange(0, head_dim, 2, dtype=np.float32)) / np.float32(head_dim))).astype(
        np.float32)
    ang = (pos * inv[None, :]).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, round_f16: bool = True) -> np.ndarray:
    """Interleaved-pair RoPE on x [..., S, D] (position = index along S).
    Returns a new fp32 array."""
    y = _c(x, np.float32).copy()
    s, d = y.shape[-2], y.shape[-1]
    bh = int(np.prod(y.shape[:-2])) if y.ndim > 2 else 1
    cos = _c(cos, np.float32)
    sin = _c(sin, np.float32)
    if cos.shape[0] < s or cos.shape[1] != d // 2:
        raise ValueError("rope table shape mismatch")
    lib().oracle_rope(_p(y, _f32p), bh, s, d, _p(cos, _f32p), _p(sin, _f32p), 1 if round_f16 else 0)
    return y


def rotate_half_perm(d: int) -> np.ndarray:
    """Channel permutation P with new[2i] = old[i], new[2i+1] = old[i + d/2].
    Interleaved RoPE on x[..., P] equals rotate-half RoPE on x, permuted by P."""
    p = np.empty(d, dtype=np.int64)
    p[0::2] = np.arange(d // 2)
    p[1::2] = np.arange(d // 2) + d // 2
    return p


# --------------------------------------------------------------------------- #
# attention
# --------------------------------------------------------------------------- #
def attention(q, k, v, causal=False, window=-1, scale=None, nthreads=None, return_lse=False):
    """softmax(scale*QK^T + mask)V in fp64 -> fp32.  q [B,Hq,Sq,D], k/v [B,Hkv,Sk,D]."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    if scale is None:
        scale = d ** -0.5
    out = np.empty((b, hq, sq, d), dtype=np.float32)
    lse = np.empty((b, hq, sq), dtype=np.float32) if return_lse else None
    rc = lib().oracle_attention(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), _p(out, _f32p),
                                _p(lse, _f32p) if lse is not None else None, b, hq, hkv, sq, sk, d, float(scale),
                                1 if causal else 0, int(window), nthreads or default_threads())
    if rc != 0:
        raise ValueError(f"oracle_attention rc={rc}")
    return (out, lse) if return_lse else out


def int8_scores(qi, ki):
    qi = _c(qi, np.int8)
    ki = _c(ki, np.int8)
    b, hq, sq, d = qi.shape
    hkv, sk = ki.shape[1], ki.shape[2]
    s = np.empty((b, hq, sq, sk), dtype=np.int32)
    rc = lib().oracle_int8_scores(_p(qi, _i8p), _p(ki, _i8p), _p(s, _i32p), b, hq, hkv, sq, sk, d)
    if rc != 0:
        raise ValueError(f"oracle_int8_scores rc={rc}")
    return s


def attention_int8(qi, ki, vi, q_scale, k_scale, v_scale, causal=False, window=-1, scale=None, block_n=64,
                   nthreads=None, v_token=None):
    """Kernel-exact INT8 emulation.  q_scale / k_scale: float or per-token array.
    v_token: per-token V scales [B, Hkv, Sk] (the library's extension; V row j
    becomes fp16(v_j * fp16(v_token_j)) before P V), or None."""
    qi = _c(qi, np.int8)
    ki = _c(ki, np.int8)
    vi = _c(vi, np.int8)
    b, hq, sq, d = qi.shape
    hkv, sk = ki.shape[1], ki.shape[2]
    if scale is None:
        scale = d ** -0.5
    qsv = _c(q_scale, np.float32) if isinstance(q_scale, np.ndarray) else None
    ksv = _c(k_scale, np.float32) if isinstance(k_scale, np.ndarray) else None
    out = np.empty((b, hq, sq, d), dtype=np.float32)
    if v_token is not None:
        vtv = _c(v_token, np.float32)
        if vtv.shape != (b, hkv, sk):
            raise ValueError(f"v_token shape {vtv.shape} != {(b, hkv, sk)}")
        rc = lib().oracle_attention_int8_vtoken(_p(qi, _i8p), _p(ki, _i8p), _p(vi, _i8p),
                                                _p(qsv, _f32p) if qsv is not None else None,
                                                _p(ksv, _f32p) if ksv is not None else None, _p(vtv, _f32p),
                                                1.0 if qsv is not None else float(q_scale),
                                                1.0 if ksv is not None else float(k_scale), float(v_scale),
                                                _p(out, _f32p), b, hq, hkv, sq, sk, d, float(scale),
                                                1 if causal else 0, int(window), int(block_n),
                                                nthreads or default_threads())
        if rc != 0:
            raise ValueError(f"oracle_attention_int8_vtoken rc={rc}")
        return out
    rc = lib().oracle_attention_int8(_p(qi, _i8p), _p(ki, _i8p), _p(vi, _i8p),
                                     _p(qsv, _f32p) if qsv is not None else None,
                                     _p(ksv, _f32p) if ksv is not None else None,
                                     1.0 if qsv is not None else float(q_scale),
                                     1.0 if ksv is not None else float(k_scale), float(v_scale), _p(out, _f32p),
                                     b, hq, hkv, sq, sk, d, float(scale), 1 if causal else 0, int(window),
                                     int(block_n), nthreads or default_threads())
    if rc != 0:
        raise ValueError(f"oracle_attention_int8 rc={rc}")
    return out


def attention_int8_gate(qd, kd, vd, causal=False, window=-1, scale=None, nthreads=None):
    """Gate-style INT8 emulation on dequantised fp32 Q/K/V (global-max P quantisation)."""
    qd = _c(qd, np.float32)
    kd = _c(kd, np.float32)
    vd = _c(vd, np.float32)
    b, hq, sq, d = qd.shape
    hkv, sk = kd.shape[1], kd.shape[2]
    if scale is None:
        scale = d ** -0.5
    out = np.empty((b, hq, sq, d), dtype=np.float32)
    rc = lib().oracle_attention_int8_gate(_p(qd, _f32p), _p(kd, _f32p), _p(vd, _f32p), _p(out, _f32p), b, hq, hkv,
                                          sq, sk, d, float(scale), 1 if causal else 0, int(window),
                                          nthreads or default_threads())
    if rc != 0:
        raise ValueError(f"oracle_attention_int8_gate rc={rc}")
    return out


# --------------------------------------------------------------------------- #
# quantisers
# --------------------------------------------------------------------------- #
def quant_pertoken(x):
    """x [..., D] -> (int8 [..., D], scale [...])."""
    x = _c(x, np.float32)
    d = x.shape[-1]
    rows = x.size // d if d else 0
    q = np.empty(x.shape, dtype=np.int8)
    s = np.empty(x.shape[:-1], dtype=np.float32)
    lib().oracle_quant_pertoken(_p(x, _f32p), rows, d, _p(q, _i8p), _p(s, _f32p))
    return q, s


def quant_perchannel(v):
    """v [B,H,S,D] -> (int8 [B,H,S,D], v_channel [B,H,D])."""
    v = _c(v, np.float32)
    b, h, s, d = v.shape
    vi = np.empty(v.shape, dtype=np.int8)
    vch = np.empty((b, h, d), dtype=np.float32)
    lib().oracle_quant_perchannel(_p(v, _f32p), b * h, s, d, _p(vi, _i8p), _p(vch, _f32p))
    return vi, vch


def quant_pertensor(x):
    x = _c(x, np.float32)
    q = np.empty(x.shape, dtype=np.int8)
    s = lib().oracle_quant_pertensor(_p(x, _f32p), x.size, _p(q, _i8p))
    return q, float(s)


# --------------------------------------------------------------------------- #
# the reference gates' input generators
# --------------------------------------------------------------------------- #
class Lcg:
    """The LCG stream of tests/hip_forward_gate.hip:31-37 (mode 0) and
    tests/hip_forward_int8qk_gate.hip:44-50 (mode 1)."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint32(seed & 0xFFFFFFFF)

    def fill(self, shape, mode: int = 0) -> np.ndarray:
        n = int(np.prod(shape))
        out = np.empty(n, dtype=np.float32)
        lib().oracle_lcg_fill(_p(out, _f32p), n, ctypes.byref(self.state), mode)
        return out.reshape(shape)
