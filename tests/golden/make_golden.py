"""Writes the golden fixtures of this directory from the CPU oracle.

    python tests/golden/make_golden.py

Each fixture is an .npz (no pickled objects) holding the inputs (fp16 or
int8, drawn from numpy's PCG64 with a fixed seed), the case parameters and
the expected outputs computed by the oracle in fp64:
  f16_<case>.npz   q, k, v [, cos, sin], out (fp32), params
  i8_<case>.npz    qi, ki, vi, q_scale, k_scale, v_scale, scores (int32),
                   out (fp32, the kernel-exact emulation), params
The reference ships no golden vectors for this path; these pin the oracle's
results so that the GPU tests compare against fixed numbers and any change to
the oracle shows up as a fixture mismatch (tests/test_golden.py).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

import oracle  # noqa: E402

# name: (b, hq, hkv, sq, sk, d, causal, window, rope, std)
F16_CASES = {
    "mha_dense_d64": (1, 2, 2, 64, 64, 64, False, -1, False, 1.0),
    "causal_gqa_rope_d128": (1, 4, 2, 80, 80, 128, True, -1, True, 1.0),
    "window_two_sided_d64": (1, 2, 2, 80, 80, 64, False, 32, False, 1.0),
    "causal_window_d64": (1, 2, 2, 80, 80, 64, True, 16, False, 1.0),
    "decode_gqa_d128": (1, 8, 2, 1, 257, 128, False, -1, False, 1.0),
    "cross_longer_keys_d32": (1, 2, 2, 40, 100, 32, True, -1, False, 1.0),
    "rows_without_keys_d64": (1, 2, 2, 50, 20, 64, True, -1, False, 1.0),
    "large_head_rope_d512": (1, 2, 2, 32, 32, 512, True, -1, True, 0.5),
    "window_rope_d256": (1, 2, 2, 64, 64, 256, False, 32, True, 0.5),
}
# name: (b, hq, hkv, sq, sk, d, causal, window, per_token)
I8_CASES = {
    "pertoken_causal_gqa_d128": (1, 4, 2, 96, 96, 128, True, -1, True),
    "pertensor_window_d64": (1, 2, 2, 80, 80, 64, False, 32, False),
}


def f16_fixture(seed, case):
    b, hq, hkv, sq, sk, d, causal, window, rope, std = case
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((b, hq, sq, d)) * std).astype(np.float16)
    k = (rng.standard_normal((b, hkv, sk, d)) * std).astype(np.float16)
    v = (rng.standard_normal((b, hkv, sk, d)) * std).astype(np.float16)
    qf, kf = q.astype(np.float32), k.astype(np.float32)
    fx = {"q": q, "k": k, "v": v}
    if rope:
        cos, sin = oracle.rope_tables(max(sq, sk), d)
        qf = oracle.rope(qf, cos, sin, round_f16=True)
        kf = oracle.rope(kf, cos, sin, round_f16=True)
        fx["cos"], fx["sin"] = cos, sin
    fx["out"] = oracle.attention(qf, kf, v.astype(np.float32), causal=causal, window=window, nthreads=1)
    fx["params"] = np.array([b, hq, hkv, sq, sk, d, int(causal), window, int(rope)], dtype=np.int64)
    fx["std"] = np.float32(std)
    return fx


def i8_fixture(seed, case):
    b, hq, hkv, sq, sk, d, causal, window, per_token = case
    rng = np.random.default_rng(seed)
    qf = rng.standard_normal((b, hq, sq, d)).astype(np.float32)
    kf = rng.standard_normal((b, hkv, sk, d)).astype(np.float32)
    vf = rng.standard_normal((b, hkv, sk, d)).astype(np.float32)
    if per_token:
        qi, qs = oracle.quant_pertoken(qf)
        ki, ks = oracle.quant_pertoken(kf)
    else:
        qi, qs = oracle.quant_pertensor(qf)
        ki, ks = oracle.quant_pertensor(kf)
    vi, vs = oracle.quant_pertensor(vf)
    fx = {"qi": qi, "ki": ki, "vi": vi,
          "q_scale": np.asarray(qs, dtype=np.float32), "k_scale": np.asarray(ks, dtype=np.float32),
          "v_scale": np.float32(vs)}
    fx["scores"] = oracle.int8_scores(qi, ki)
    fx["out"] = oracle.attention_int8(qi, ki, vi, qs, ks, vs, causal=causal, window=window, nthreads=1)
    fx["params"] = np.array([b, hq, hkv, sq, sk, d, int(causal), window, int(per_token)], dtype=np.int64)
    return fx


def main() -> int:
    oracle.build()
    for i, (name, case) in enumerate(F16_CASES.items()):
        np.savez_compressed(HERE / f"f16_{name}.npz", **f16_fixture(1000 + i, case))
    for i, (name, case) in enumerate(I8_CASES.items()):
        np.savez_compressed(HERE / f"i8_{name}.npz", **i8_fixture(2000 + i, case))
    print(f"wrote {len(F16_CASES) + len(I8_CASES)} fixtures to {HERE}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
