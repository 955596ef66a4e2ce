"""The HIP path on the committed golden fixtures (tests/golden/*.npz): FP16
outputs within the FP16 bars, INT8 int32 scores bit-exact and outputs within
the INT8 bar of the stored emulation."""
from pathlib import Path

import numpy as np
import pytest
import torch

from tests.gpu_util import I8_MAX_ABS, assert_f16_parity, errors, forward_raw, lib, log, stream_ptr

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
F16 = sorted(GOLDEN.glob("f16_*.npz"))
I8 = sorted(GOLDEN.glob("i8_*.npz"))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("path", F16, ids=[p.stem for p in F16])
def test_f16_golden(gpu, path):
    fx = load(path)
    log(f"[golden] {path.stem}")
    b, hq, hkv, sq, sk, d, causal, window, rope = (int(x) for x in fx["params"])
    q, k, v = (torch.from_numpy(fx[n]).to(gpu) for n in ("q", "k", "v"))
    cos = torch.from_numpy(fx["cos"]).to(gpu) if rope else None
    sin = torch.from_numpy(fx["sin"]).to(gpu) if rope else None
    out = torch.empty_like(q)
    assert forward_raw(q, k, v, out, bool(causal), window, cos, sin) == 0
    torch.cuda.synchronize()
    assert_f16_parity(out.float().cpu().numpy(), fx["out"], path.stem)


@pytest.mark.parametrize("path", I8, ids=[p.stem for p in I8])
def test_i8_golden(gpu, path):
    import ctypes

    fx = load(path)
    log(f"[golden] {path.stem}")
    b, hq, hkv, sq, sk, d, causal, window, per_token = (int(x) for x in fx["params"])
    qi, ki, vi = (torch.from_numpy(fx[n]).to(gpu) for n in ("qi", "ki", "vi"))
    scores = torch.empty(b, hq, sq, sk, dtype=torch.int32, device=gpu)
    qs, ks = qi.stride(), ki.stride()
    L = lib()
    assert L.rdna_int8_qk_scores(qi.data_ptr(), ki.data_ptr(), ctypes.c_void_p(scores.data_ptr()), qs[0], qs[1], qs[2],
                                 ks[0], ks[1], ks[2], b, hq, hkv, sq, sk, d, stream_ptr()) == 0
    out = torch.empty(b, hq, sq, d, dtype=torch.float16, device=gpu)
    if per_token:
        qv = torch.from_numpy(fx["q_scale"]).to(gpu)
        kv = torch.from_numpy(fx["k_scale"]).to(gpu)
        q_s, k_s, qp, kp = 1.0, 1.0, qv.data_ptr(), kv.data_ptr()
    else:
        q_s, k_s, qp, kp = float(fx["q_scale"]), float(fx["k_scale"]), None, None
    vs, os_ = vi.stride(), out.stride()
    rc = L.rdna_attention_forward_int8qk(qi.data_ptr(), ki.data_ptr(), vi.data_ptr(), out.data_ptr(),
                                         qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2],
                                         os_[0], os_[1], os_[2], b, hq, hkv, sq, sk, d, d ** -0.5, q_s, k_s,
                                         float(fx["v_scale"]), qp, kp, 1 if causal else 0, window, stream_ptr())
    assert rc == 0
    torch.cuda.synchronize()
    assert np.array_equal(scores.cpu().numpy(), fx["scores"])
    mx, _, _ = errors(out.float().cpu().numpy(), fx["out"])
    assert mx <= I8_MAX_ABS, f"{path.stem}: max_abs={mx:.3e}"
