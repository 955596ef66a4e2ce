"""rdnattention -- FlashAttention-2 forward for MI355X (gfx950), a drop-in
for the ``rdnattention`` Python package of dmonkman/RDNAttention.

The public surface is the reference's (rdnattention/__init__.py:360-363):
``flash_attn``, ``flash_attn_int8qk``, ``flash_attn_int8qk_quantized``,
``quantize_int8_perchannel_v``, ``quantize_int8_qk_pertoken``,
``has_device``, ``RDNAttentionError``, ``SUPPORTED_HEAD_DIMS``,
``SUPPORTED_HEAD_DIMS_INT8`` and ``__version__``, with the same argument
checks and exception types.  Every call goes through ``librdnattention.so``
(HIP kernels for gfx950) on torch's current stream; there is no CPU
fallback: a missing library raises ``RDNAttentionError``.

    >>> import torch
    >>> from rdnattention import flash_attn
    >>> q = torch.randn(1, 8, 512, 64, dtype=torch.float16, device="cuda")
    >>> k = torch.randn(1, 8, 512, 64, dtype=torch.float16, device="cuda")
    >>> v = torch.randn(1, 8, 512, 64, dtype=torch.float16, device="cuda")
    >>> out = flash_attn(q, k, v, is_causal=True)
"""
from __future__ import annotations

import ctypes
import logging
import os
import platform
from pathlib import Path

logger = logging.getLogger(__name__)

__version__ = "0.1.0"

_lib = None

SUPPORTED_HEAD_DIMS = tuple(range(32, 513, 32))
SUPPORTED_HEAD_DIMS_INT8 = (64, 128)

PATH_AUTO = 0
PATH_PREFILL = 1
PATH_SPLITK = 2


class RDNAttentionError(Exception):
    """Raised for any rdnattention library error."""


def _library_candidates() -> list:
    """Search order after RDNATTENTION_LIB (rdnattention/__init__.py:54-61): the
    development build build/librdnattention.so and the packaged
    lib/librdnattention.so, the development build first in a source checkout
    (where the native sources rdnattention_amd/csrc sit next to the package),
    so that a stale lib/ never shadows a rebuild."""
    here = Path(__file__).resolve().parent
    packaged = here / "lib" / "librdnattention.so"
    dev = here.parent / "build" / "librdnattention.so"
    in_source_tree = (here.parent / "rdnattention_amd" / "csrc").is_dir()
    return [dev, packaged] if in_source_tree else [packaged, dev]


def _find_library() -> Path:
    """RDNATTENTION_LIB, else the candidates of _library_candidates()
    (rdnattention/__init__.py:37-73; Linux only: this build targets ROCm)."""
    if platform.system() != "Linux":
        raise RDNAttentionError(f"Unsupported platform: {platform.system()} (this build targets Linux/ROCm)")
    override = os.environ.get("RDNATTENTION_LIB")
    if override:
        path = Path(override)
        if not path.exists():
            raise RDNAttentionError(f"RDNATTENTION_LIB points at a missing file: {path}")
        logger.debug("Loading library from RDNATTENTION_LIB=%s", path)
        return path
    candidates = _library_candidates()
    for path in candidates:
        if path.exists():
            others = [c for c in candidates if c != path and c.exists()]
            if others and path == candidates[0] and path.parent.name == "build":
                logger.warning("Ignoring the packaged %s: this is a source checkout, so %s takes priority. "
                               "Delete lib/ to silence this.", others[0], path)
            logger.debug("Loading library from %s", path)
            return path
    raise RDNAttentionError(
        "Could not find the rdnattention library (librdnattention.so). Build it first "
        "(python -m rdnattention._build), or install the wheel.\n"
        f"Searched: {[str(p) for p in candidates]}")


_VP = ctypes.c_void_p
_I64 = ctypes.c_int64
_U32 = ctypes.c_uint32
_I32 = ctypes.c_int32
_F32 = ctypes.c_float

_FWD_ARGS = [_VP] * 6 + [_I64] * 12 + [_U32] * 6 + [_F32, _I32, _I32, _I32]
_I8_ARGS = [_VP] * 4 + [_I64] * 12 + [_U32] * 6 + [_F32] * 4 + [_VP, _VP, _I32, _I32, _VP]


def _lib_handle():
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(str(_find_library()))
        lib.rdna_has_device.argtypes = []
        lib.rdna_has_device.restype = _I32
        lib.rdna_get_error.argtypes = []
        lib.rdna_get_error.restype = ctypes.c_char_p
        lib.rdna_attention_forward.argtypes = _FWD_ARGS + [_VP]
        lib.rdna_attention_forward.restype = _I32
        lib.rdna_attention_forward_path.argtypes = _FWD_ARGS + [_I32, _VP]
        lib.rdna_attention_forward_path.restype = _I32
        try:  # absent from libraries built before it existed (RDNATTENTION_LIB may name one)
            lib.rdna_attention_forward_noalloc.argtypes = _FWD_ARGS + [_VP]
            lib.rdna_attention_forward_noalloc.restype = _I32
        except AttributeError:
            pass
        lib.rdna_attention_forward_int8qk.argtypes = _I8_ARGS
        lib.rdna_attention_forward_int8qk.restype = _I32
        lib.rdna_attention_forward_int8qk_vchannel.argtypes = _I8_ARGS[:-3] + [_VP] + _I8_ARGS[-3:]
        lib.rdna_attention_forward_int8qk_vchannel.restype = _I32
        lib.rdna_attention_forward_int8qk_vtoken.argtypes = _I8_ARGS[:-3] + [_VP] + _I8_ARGS[-3:]
        lib.rdna_attention_forward_int8qk_vtoken.restype = _I32
        lib.rdna_quantize_int8.argtypes = [_VP, _I32] + [_I64] * 3 + [_U32] * 4 + [_I32, _VP, _VP, _VP, _VP, _VP]
        lib.rdna_quantize_int8.restype = _I32
        lib.rdna_int8_qk_scores.argtypes = [_VP] * 3 + [_I64] * 6 + [_U32] * 6 + [_VP]
        lib.rdna_int8_qk_scores.restype = _I32
        try:  # absent from libraries built before it existed
            lib.rdna_scratch_trim.argtypes = []
            lib.rdna_scratch_trim.restype = _I32
            lib.rdna_scratch_stats.argtypes = [_I32, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(_I64),
                                               ctypes.POINTER(_I64)]
            lib.rdna_scratch_stats.restype = _I32
        except AttributeError:
            pass
        lib.rdna_kernel_timer_enable.argtypes = [_I32]
        lib.rdna_kernel_timer_enable.restype = _I32
        lib.rdna_kernel_timer_read.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I64)]
        lib.rdna_kernel_timer_read.restype = _I32
        lib.rdna_version.argtypes = []
        lib.rdna_version.restype = ctypes.c_char_p
        _lib = lib
    return _lib


def library_path() -> Path:
    return Path(_lib_handle()._name)


def has_device() -> bool:
    """Whether a usable HIP device is present."""
    return _lib_handle().rdna_has_device() == 1


def last_error() -> str:
    return _lib_handle().rdna_get_error().decode()


def _validate_inputs(query, key, value, expected_dtype) -> None:
    # rdnattention/__init__.py:138-155
    import torch

    if not isinstance(query, torch.Tensor):
        raise TypeError("requires torch.Tensor inputs (GPU tensors already on this device)")
    for name, t in (("query", query), ("key", key), ("value", value)):
        if not isinstance(t, torch.Tensor):
            raise TypeError("requires torch.Tensor inputs (GPU tensors already on this device)")
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a HIP device")
        if t.dtype != expected_dtype:
            raise ValueError(f"{name} must be {expected_dtype}, got {t.dtype}")
        if t.dim() != 4:
            raise ValueError(f"{name} must be 4D [batch, heads, seq, head_dim], got shape {tuple(t.shape)}")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous - call .contiguous() first")
    _check_shapes(query, key, value)


def _check_shapes(query, key, value) -> None:
    """The shape relations every kernel relies on: one batch size, V shaped
    like K, one head_dim, and a whole number of query heads per kv head.  The
    first and last are the reference's checks (rdnattention/__init__.py:151-
    155); the kernels would read past the end of a smaller K/V otherwise, so
    the middle two are added here."""
    if query.shape[0] != key.shape[0] or query.shape[0] != value.shape[0]:
        raise ValueError(f"Batch size must match: Q={query.shape}, K={key.shape}, V={value.shape}")
    if tuple(key.shape) != tuple(value.shape):
        raise ValueError(f"key and value must have the same shape: K={tuple(key.shape)}, V={tuple(value.shape)}")
    if key.shape[3] != query.shape[3]:
        raise ValueError(f"key head_dim ({key.shape[3]}) must equal query head_dim ({query.shape[3]})")
    if key.shape[1] == 0 or query.shape[1] % key.shape[1] != 0:
        raise ValueError(f"Q heads ({query.shape[1]}) must be a multiple of K heads ({key.shape[1]})")


def _check_head_dim(head_dim: int, who: str, allowed=SUPPORTED_HEAD_DIMS):
    # rdnattention/__init__.py:158-162
    if head_dim not in allowed:
        raise RDNAttentionError(
            f"{who}: head_dim {head_dim} not supported "
            f"(multiples of 32 from {allowed[0]} to {allowed[-1]})")


def _rope_ptrs(rot_cos, rot_sin, query, seq_len, key_seq_len, head_dim):
    """Validates the angle tables (rdnattention/__init__.py:165-192).
    Returns (cos_ptr, sin_ptr, has_rope)."""
    import torch

    if rot_cos is None and rot_sin is None:
        return None, None, 0
    if rot_cos is None or rot_sin is None:
        raise ValueError("pass both rot_cos and rot_sin, or neither")
    rows = max(seq_len, key_seq_len)
    for name, t in (("rot_cos", rot_cos), ("rot_sin", rot_sin)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if t.device != query.device:
            raise ValueError(f"{name} must be on the same device as query")
        if t.dtype != torch.float32:
            raise ValueError(f"{name} must be float32, got {t.dtype}")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous - call .contiguous() first")
        if t.dim() != 2:
            raise ValueError(f"{name} must be 2D [positions, head_dim // 2], got {tuple(t.shape)}")
        if t.shape[1] != head_dim // 2:
            raise ValueError(f"{name} must have head_dim // 2 = {head_dim // 2} columns, got {t.shape[1]}")
        if t.shape[0] < rows:
            raise ValueError(f"{name} needs at least max(seq_len, key_seq_len) = {rows} rows, got {t.shape[0]}")
    return rot_cos.data_ptr(), rot_sin.data_ptr(), 1


def _stream():
    import torch

    return torch.cuda.current_stream().cuda_stream


def flash_attn(query, key, value, is_causal: bool = False, window_size: int = -1, rot_cos=None, rot_sin=None):
    """FlashAttention-2 forward in fp16 (rdnattention/__init__.py:195-238).

    query/key/value: contiguous float16 [batch, heads, seq, head_dim] on a HIP
    device, head_dim in SUPPORTED_HEAD_DIMS; key/value may have fewer heads
    (GQA/MQA, an exact divisor) and a different sequence length (decode,
    cross-attention; causal aligns to the end of the keys).  rot_cos/rot_sin:
    float32 [max(seq_len, key_seq_len), head_dim // 2] RoPE tables applied to
    Q and K inside the kernel (channels 2i, 2i+1 rotate by column i).
    The softmax scale is 1/sqrt(head_dim).  Returns a new tensor like query.
    """
    import torch

    _validate_inputs(query, key, value, torch.float16)
    _check_head_dim(query.shape[-1], "flash_attn")
    if not has_device():
        raise RDNAttentionError("no usable HIP device found")
    batch, heads, seq_len, head_dim = query.shape
    _, kv_heads, key_seq_len, _ = key.shape
    cos_ptr, sin_ptr, has_rope = _rope_ptrs(rot_cos, rot_sin, query, seq_len, key_seq_len, head_dim)
    output = torch.empty_like(query)
    if output.numel() == 0:
        return output
    qs, ks, vs, os_ = query.stride(), key.stride(), value.stride(), output.stride()
    result = _lib_handle().rdna_attention_forward(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), output.data_ptr(), cos_ptr, sin_ptr,
        qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os_[0], os_[1], os_[2],
        batch, heads, kv_heads, seq_len, key_seq_len, head_dim,
        head_dim ** -0.5, 1 if is_causal else 0, has_rope, window_size, _stream())
    if result != 0:
        raise RDNAttentionError(f"flash_attn failed: {last_error()}")
    return output


def attention_forward_into(query, key, value, output, *, is_causal: bool = False, window_size: int = -1,
                           rot_cos=None, rot_sin=None, scale=None, path: int = PATH_AUTO) -> None:
    """FP16 forward written into `output`, for strided tensors and explicit
    kernel paths -- the direct C-ABI call the reference's own tools make
    through ctypes (tests/rope.py:9-27, tests/benchmark.py:232-263).

    query/key/value/output: float16 [batch, heads, seq, head_dim] views whose
    head_dim axis is contiguous (any batch/head/seq strides that are multiples
    of 8 elements, e.g. K/V sliced from a [B, S, 2, Hkv, D] cache).
    `scale` defaults to 1/sqrt(head_dim); `path` is PATH_AUTO, PATH_PREFILL or
    PATH_SPLITK.  Asynchronous on torch's current stream."""
    import torch

    for name, t in (("query", query), ("key", key), ("value", value), ("output", output)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if t.dtype != torch.float16 or t.dim() != 4 or not t.is_cuda:
            raise ValueError(f"{name} must be a 4D float16 HIP tensor")
        if t.stride(-1) != 1:
            raise ValueError(f"{name} must have a contiguous head_dim axis")
    if output.shape != query.shape:
        raise ValueError("output must have the shape of query")
    _check_shapes(query, key, value)
    batch, heads, seq_len, head_dim = query.shape
    _, kv_heads, key_seq_len, _ = key.shape
    cos_ptr, sin_ptr, has_rope = _rope_ptrs(rot_cos, rot_sin, query, seq_len, key_seq_len, head_dim)
    qs, ks, vs, os_ = query.stride(), key.stride(), value.stride(), output.stride()
    result = _lib_handle().rdna_attention_forward_path(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), output.data_ptr(), cos_ptr, sin_ptr,
        qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os_[0], os_[1], os_[2],
        batch, heads, kv_heads, seq_len, key_seq_len, head_dim,
        float(head_dim ** -0.5 if scale is None else scale), 1 if is_causal else 0, has_rope, int(window_size),
        int(path), _stream())
    if result != 0:
        raise RDNAttentionError(f"attention_forward_into failed: {last_error()}")


def flash_attn_int8qk(query, key, value, q_scale, k_scale, v_scale: float, is_causal: bool = False,
                      window_size: int = -1):
    """INT8 attention, both GEMMs (rdnattention/__init__.py:241-300).

    query/key/value: contiguous int8 [batch, heads, seq, head_dim], head_dim
    in SUPPORTED_HEAD_DIMS_INT8.  q_scale/k_scale: float, or float32 tensors
    of per-token scales shaped (batch, heads, seq_len) / (batch, kv_heads,
    key_seq_len); v_scale: float.  Output float16.  No RoPE.
    """
    import torch

    _validate_inputs(query, key, value, torch.int8)
    heads, kv_heads_ = query.shape[1], key.shape[1]
    if kv_heads_ == 0 or heads % kv_heads_ != 0:
        raise RDNAttentionError(
            f"flash_attn_int8qk: query heads ({heads}) must be a positive multiple of key/value heads ({kv_heads_})")
    _check_head_dim(query.shape[-1], "flash_attn_int8qk", allowed=SUPPORTED_HEAD_DIMS_INT8)
    if not has_device():
        raise RDNAttentionError("no usable HIP device found")
    batch, heads, seq_len, head_dim = query.shape
    _, kv_heads, key_seq_len, _ = key.shape

    def _scale_arg(x, name, want):
        if not isinstance(x, torch.Tensor):
            return float(x), None
        t = x.to(dtype=torch.float32, device=query.device).contiguous()
        if tuple(t.shape) != want:
            raise RDNAttentionError(f"flash_attn_int8qk: {name} tensor must be {want}, got {tuple(t.shape)}")
        return 1.0, t

    q_scalar, q_vec = _scale_arg(q_scale, "q_scale", (batch, heads, seq_len))
    k_scalar, k_vec = _scale_arg(k_scale, "k_scale", (batch, kv_heads, key_seq_len))
    output = torch.empty(query.shape, dtype=torch.float16, device=query.device)
    if output.numel() == 0:
        return output
    qs, ks, vs, os_ = query.stride(), key.stride(), value.stride(), output.stride()
    result = _lib_handle().rdna_attention_forward_int8qk(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), output.data_ptr(),
        qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os_[0], os_[1], os_[2],
        batch, heads, kv_heads, seq_len, key_seq_len, head_dim,
        head_dim ** -0.5, q_scalar, k_scalar, float(v_scale),
        q_vec.data_ptr() if q_vec is not None else None, k_vec.data_ptr() if k_vec is not None else None,
        1 if is_causal else 0, window_size, _stream())
    if result != 0:
        raise RDNAttentionError(f"flash_attn_int8qk failed: {last_error()}")
    return output


def attention_int8_forward_into(query, key, value, output, q_scale, k_scale, v_scale: float, *,
                                is_causal: bool = False, window_size: int = -1, scale=None,
                                v_channel=None, v_token=None) -> None:
    """INT8 forward written into a preallocated float16 `output` (the raw
    rdna_attention_forward_int8qk call, src/c_api.cpp:116-195).

    query/key/value: int8 [batch, heads, seq, head_dim] views with a
    contiguous head_dim axis and batch/head/seq strides that are multiples of
    16 elements.  q_scale/k_scale: floats, or contiguous float32 device
    tensors of per-token scales [batch, heads, seq_len] /
    [batch, kv_heads, key_seq_len].  v_channel: optional contiguous float32
    device tensor [batch, kv_heads, head_dim] of per-channel V scales applied
    in the kernel (rdna_attention_forward_int8qk_vchannel).  v_token:
    optional contiguous float32 device tensor [batch, kv_heads, key_seq_len]
    of per-token V scales, each V row dequantised by its own scale in the
    kernel (rdna_attention_forward_int8qk_vtoken; exclusive with v_channel).
    Asynchronous on torch's current stream."""
    import torch

    for name, t in (("query", query), ("key", key), ("value", value)):
        if not isinstance(t, torch.Tensor) or t.dtype != torch.int8 or t.dim() != 4 or not t.is_cuda:
            raise ValueError(f"{name} must be a 4D int8 HIP tensor")
    if output.dtype != torch.float16 or output.shape != query.shape or not output.is_cuda:
        raise ValueError("output must be a float16 HIP tensor with the shape of query")
    _check_shapes(query, key, value)
    batch, heads, seq_len, head_dim = query.shape
    _, kv_heads, key_seq_len, _ = key.shape

    def _scale_arg(x, name, want):
        if not isinstance(x, torch.Tensor):
            return float(x), None
        if x.dtype != torch.float32 or not x.is_contiguous() or tuple(x.shape) != want or not x.is_cuda:
            raise ValueError(f"{name} must be a contiguous float32 HIP tensor of shape {want}")
        return 1.0, x

    q_scalar, q_vec = _scale_arg(q_scale, "q_scale", (batch, heads, seq_len))
    k_scalar, k_vec = _scale_arg(k_scale, "k_scale", (batch, kv_heads, key_seq_len))
    qs, ks, vs, os_ = query.stride(), key.stride(), value.stride(), output.stride()
    args = [query.data_ptr(), key.data_ptr(), value.data_ptr(), output.data_ptr(),
            qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os_[0], os_[1], os_[2],
            batch, heads, kv_heads, seq_len, key_seq_len, head_dim,
            float(head_dim ** -0.5 if scale is None else scale), q_scalar, k_scalar, float(v_scale),
            q_vec.data_ptr() if q_vec is not None else None, k_vec.data_ptr() if k_vec is not None else None]
    tail = [1 if is_causal else 0, int(window_size), _stream()]
    if v_channel is not None and v_token is not None:
        raise ValueError("pass v_channel or v_token, not both")
    if v_token is not None:
        want = (batch, kv_heads, key_seq_len)
        if (not isinstance(v_token, torch.Tensor) or v_token.dtype != torch.float32
                or not v_token.is_contiguous() or tuple(v_token.shape) != want or not v_token.is_cuda):
            raise ValueError(f"v_token must be a contiguous float32 HIP tensor of shape {want}")
        result = _lib_handle().rdna_attention_forward_int8qk_vtoken(*args, v_token.data_ptr(), *tail)
    elif v_channel is None:
        result = _lib_handle().rdna_attention_forward_int8qk(*args, *tail)
    else:
        want = (batch, kv_heads, head_dim)
        if (not isinstance(v_channel, torch.Tensor) or v_channel.dtype != torch.float32
                or not v_channel.is_contiguous() or tuple(v_channel.shape) != want or not v_channel.is_cuda):
            raise ValueError(f"v_channel must be a contiguous float32 HIP tensor of shape {want}")
        result = _lib_handle().rdna_attention_forward_int8qk_vchannel(*args, v_channel.data_ptr(), *tail)
    if result != 0:
        raise RDNAttentionError(f"attention_int8_forward_into failed: {last_error()}")


def trim_scratch() -> None:
    """Returns the scratch memory the library keeps for reuse to the devices:
    the buffers cached per (device, stream, use) for RoPE-rotated K copies,
    split-K partials and quantiser partials (each grown to the largest call so
    far; at most 1 GiB per device), and the free blocks of the devices'
    default memory pools; e.g. before handing memory to another allocator.
    Synchronises the devices.  An extension; the reference allocates nothing."""
    if _lib_handle().rdna_scratch_trim() != 0:
        raise RDNAttentionError(f"trim_scratch failed: {last_error()}")


def scratch_stats(device: int = 0) -> dict:
    """The scratch cache of HIP device `device`: {"cached_bytes", "entries",
    "allocations"}, the last being the allocator calls the library has made
    for that device's scratch since it was loaded.  An extension."""
    nbytes, entries, allocs = ctypes.c_uint64(), _I64(), _I64()
    if _lib_handle().rdna_scratch_stats(int(device), ctypes.byref(nbytes), ctypes.byref(entries),
                                        ctypes.byref(allocs)) != 0:
        raise RDNAttentionError(f"scratch_stats failed: {last_error()}")
    return {"cached_bytes": nbytes.value, "entries": entries.value, "allocations": allocs.value}


class KernelTimer:
    """Context manager timing the library's main attention kernels with HIP
    events recorded on their launch streams (rdna_kernel_timer_enable/_read):
    RoPE pre-rotation and split-K combine launches are not included.  After
    the block, `total_ms` and `launches` hold the summed kernel time and the
    number of timed launches; `mean_ms` their ratio."""

    def __init__(self):
        self.total_ms = 0.0
        self.launches = 0

    @property
    def mean_ms(self) -> float:
        return self.total_ms / self.launches if self.launches else float("nan")

    def __enter__(self):
        _lib_handle().rdna_kernel_timer_enable(1)
        return self

    def __exit__(self, *exc):
        lib = _lib_handle()
        ms = ctypes.c_double(0.0)
        n = _I64(0)
        rc = lib.rdna_kernel_timer_read(ctypes.byref(ms), ctypes.byref(n))
        lib.rdna_kernel_timer_enable(0)
        if rc != 0 and exc[0] is None:
            raise RDNAttentionError("kernel timer: a HIP event could not be created, recorded or read")
        self.total_ms, self.launches = ms.value, n.value
        return False


def _quantize_gpu(x, per_channel: bool, rot_cos=None, rot_sin=None):
    """rdna_quantize_int8 on a HIP tensor [B, H, S, D]: (int8 [B, H, S, D]
    contiguous, float32 scales [B, H, S] per token or [B, H, D] per channel),
    bit-identical to the torch formulas of the reference wrapper.  With
    rot_cos/rot_sin (per token only) the rows are RoPE-rotated first, with the
    FP16 attention path's arithmetic."""
    import torch

    if x.dim() != 4:
        raise ValueError(f"expected a 4D [batch, heads, seq, head_dim] tensor, got shape {tuple(x.shape)}")
    if x.dtype not in (torch.float16, torch.float32):
        x = x.float()
    dt = 0 if x.dtype == torch.float16 else 1
    mult = 8 if dt == 0 else 4
    if x.stride(-1) != 1 or any(st % mult for st in x.stride()[:3]) or x.data_ptr() % 16:
        x = x.contiguous()
    b, h, s, d = x.shape
    if d % 8 != 0 or d > 512:
        raise RDNAttentionError(f"GPU quantiser: head_dim {d} must be a multiple of 8 up to 512")
    cos_ptr, sin_ptr, has_rope = _rope_ptrs(rot_cos, rot_sin, x, s, s, d)
    if has_rope and per_channel:
        raise ValueError("RoPE applies to the per-token (query/key) quantiser only")
    q = torch.empty((b, h, s, d), dtype=torch.int8, device=x.device)
    sc = torch.ones((b, h, d) if per_channel else (b, h, s), dtype=torch.float32, device=x.device)
    if q.numel() == 0:
        return q, sc
    st = x.stride()
    rc = _lib_handle().rdna_quantize_int8(x.data_ptr(), dt, st[0], st[1], st[2], b, h, s, d, 1 if per_channel else 0,
                                          cos_ptr, sin_ptr, q.data_ptr(), sc.data_ptr(), _stream())
    if rc != 0:
        raise RDNAttentionError(f"quantisation failed: {last_error()}")
    return q, sc


def quantize_int8_perchannel_v(query, key, value):
    """(qi, ki, vi, q_scale, k_scale, v_scale, v_channel) with per-tensor Q/K
    scales and one V scale per (batch, kv head, channel); v_scale = 1.0
    (rdnattention/__init__.py:303-324).  Attention is linear in V, so
    multiplying the output by v_channel undoes the V scaling exactly.

    On HIP tensors the per-channel V pass runs as a library kernel
    (rdna_quantize_int8); the per-tensor Q/K scales stay torch reductions.
    CPU tensors go through the same formulas in torch."""
    import torch

    def per_tensor(x):
        s = x.abs().max().item() / 127.0
        s = s if s != 0.0 else 1.0
        return torch.clamp(torch.round(x / s), -127, 127).to(torch.int8), s

    qi, q_scale = per_tensor(query.float())
    ki, k_scale = per_tensor(key.float())
    if value.is_cuda:
        vi, v_channel = _quantize_gpu(value, per_channel=True)
        return qi, ki, vi, q_scale, k_scale, 1.0, v_channel
    v = value.float()
    v_channel = v.abs().amax(dim=-2, keepdim=True) / 127.0
    v_channel = torch.where(v_channel == 0, torch.ones_like(v_channel), v_channel)
    vi = torch.clamp(torch.round(v / v_channel), -127, 127).to(torch.int8)
    return qi, ki, vi, q_scale, k_scale, 1.0, v_channel.squeeze(-2)


def _rope_torch(x, rot_cos, rot_sin):
    """RoPE of a [B, H, S, D] tensor in torch (interleaved pairs, position =
    row index, fp32 arithmetic, the result in x's dtype when that is fp16),
    for CPU tensors; the GPU quantiser fuses the same rotation."""
    import torch

    xf = x.float()
    n = x.shape[-2]
    c = rot_cos[:n].to(xf.device)
    sn = rot_sin[:n].to(xf.device)
    a, b = xf[..., 0::2], xf[..., 1::2]
    y = torch.empty_like(xf)
    y[..., 0::2] = a * c - b * sn
    y[..., 1::2] = a * sn + b * c
    return y.to(torch.float16) if x.dtype == torch.float16 else y


def quantize_int8_qk_pertoken(query, key, rot_cos=None, rot_sin=None):
    """(qi, ki, q_scale, k_scale) with one fp32 scale per (batch, head, row)
    (rdnattention/__init__.py:327-343).  HIP tensors are quantised by a
    library kernel (rdna_quantize_int8), bit-identical to the torch formulas
    used for CPU tensors.

    rot_cos/rot_sin (an extension; the reference has no INT8 RoPE): fp32
    [positions, head_dim // 2] tables as for flash_attn.  Query and key rows
    are RoPE-rotated, as the FP16 path rotates them, before quantisation."""
    import torch

    if query.is_cuda and key.is_cuda:
        qi, q_scale = _quantize_gpu(query, per_channel=False, rot_cos=rot_cos, rot_sin=rot_sin)
        ki, k_scale = _quantize_gpu(key, per_channel=False, rot_cos=rot_cos, rot_sin=rot_sin)
        return qi, ki, q_scale, k_scale
    if (rot_cos is None) != (rot_sin is None):
        raise ValueError("pass both rot_cos and rot_sin, or neither")
    if rot_cos is not None:
        query = _rope_torch(query, rot_cos, rot_sin)
        key = _rope_torch(key, rot_cos, rot_sin)

    def per_token(x):
        x = x.float()
        s = x.abs().amax(dim=-1, keepdim=True) / 127.0
        s = torch.where(s == 0, torch.ones_like(s), s)
        return torch.clamp(torch.round(x / s), -127, 127).to(torch.int8), s.squeeze(-1).contiguous()

    qi, q_scale = per_token(query)
    ki, k_scale = per_token(key)
    return qi, ki, q_scale, k_scale


def quantize_int8_pertoken_v(value):
    """(vi, v_token): V quantised with one fp32 scale per (batch, head, row),
    the per-token formula of quantize_int8_qk_pertoken (an extension; the
    reference has no per-token V scale).  Use with attention_int8_forward_into
    (v_token=...) or flash_attn_int8qk_quantized(v_per_token=True)."""
    import torch

    if value.is_cuda:
        return _quantize_gpu(value, per_channel=False)
    x = value.float()
    s = x.abs().amax(dim=-1, keepdim=True) / 127.0
    s = torch.where(s == 0, torch.ones_like(s), s)
    return torch.clamp(torch.round(x / s), -127, 127).to(torch.int8), s.squeeze(-1).contiguous()


def flash_attn_int8qk_quantized(query, key, value, is_causal: bool = False, window_size: int = -1, rot_cos=None,
                                rot_sin=None, v_per_token: bool = False):
    """INT8 attention from ordinary fp16/fp32 Q/K/V (rdnattention/__init__.py:346-357):
    per-token Q/K scales and a per-channel V scale.

    rot_cos/rot_sin (an extension; the reference has no INT8 RoPE): fp32
    [positions, head_dim // 2] tables as for flash_attn.  Q and K are rotated
    inside the per-token quantiser (the FP16 path's arithmetic), so RoPE costs
    no extra pass.

    Three quantiser kernels and one attention kernel: the per-channel V
    rescale is applied in the attention kernel's epilogue
    (rdna_attention_forward_int8qk_vchannel) instead of a separate pass over
    the output, and the per-tensor Q/K quantisation the reference computes and
    discards is skipped.  The output is rounded to fp16 once (the reference
    rounds the kernel output, then the rescaled product).

    Differs from the reference in one more respect: v_channel is indexed by
    the kv head of each query head, so grouped-query inputs with
    1 < kv_heads < heads work (the reference's broadcast raises there).

    v_per_token (an extension): V is quantised per token instead of per
    channel, and the kernel dequantises each V row by its scale
    (rdna_attention_forward_int8qk_vtoken)."""
    import torch

    for name, t in (("query", query), ("key", key), ("value", value)):
        if not isinstance(t, torch.Tensor):
            raise TypeError("requires torch.Tensor inputs (GPU tensors already on this device)")
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a HIP device")
        if t.dim() != 4:
            raise ValueError(f"{name} must be 4D [batch, heads, seq, head_dim], got shape {tuple(t.shape)}")
    heads, kv_heads = query.shape[1], key.shape[1]
    if kv_heads == 0 or heads % kv_heads != 0:
        raise RDNAttentionError(
            f"flash_attn_int8qk: query heads ({heads}) must be a positive multiple of key/value heads ({kv_heads})")
    _check_shapes(query, key, value)
    _check_head_dim(query.shape[-1], "flash_attn_int8qk", allowed=SUPPORTED_HEAD_DIMS_INT8)
    if not has_device():
        raise RDNAttentionError("no usable HIP device found")
    _rope_ptrs(rot_cos, rot_sin, query, query.shape[2], key.shape[2], query.shape[3])
    qi, q_scale = _quantize_gpu(query, per_channel=False, rot_cos=rot_cos, rot_sin=rot_sin)
    ki, k_scale = _quantize_gpu(key, per_channel=False, rot_cos=rot_cos, rot_sin=rot_sin)
    vi, v_sc = _quantize_gpu(value, per_channel=not v_per_token)
    output = torch.empty(query.shape, dtype=torch.float16, device=query.device)
    if output.numel() == 0:
        return output
    attention_int8_forward_into(qi, ki, vi, output, q_scale, k_scale, 1.0, is_causal=is_causal,
                                window_size=window_size, v_channel=None if v_per_token else v_sc,
                                v_token=v_sc if v_per_token else None)
    return output


__all__ = ["flash_attn", "flash_attn_int8qk", "flash_attn_int8qk_quantized", "quantize_int8_perchannel_v",
           "quantize_int8_qk_pertoken", "has_device", "RDNAttentionError", "SUPPORTED_HEAD_DIMS",
           "SUPPORTED_HEAD_DIMS_INT8", "__version__"]
