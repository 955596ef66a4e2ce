"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py) against the oracle and against closed forms.

The oracle must reproduce every fixture exactly; a change to the oracle's
arithmetic fails here first.  The dense fixture is also checked against a
plain numpy float64 softmax(QK^T/sqrt(d))V, and the int8 scores against
numpy's int64 product, so the fixtures are pinned independently of the oracle.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
F16 = sorted(GOLDEN.glob("f16_*.npz"))
I8 = sorted(GOLDEN.glob("i8_*.npz"))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fixtures_present():
    assert len(F16) >= 9 and len(I8) >= 2


@pytest.mark.parametrize("path", F16, ids=[p.stem for p in F16])
def test_f16_fixture_reproduced_by_oracle(oracle_lib, path):
    fx = load(path)
    b, hq, hkv, sq, sk, d, causal, window, rope = (int(x) for x in fx["params"])
    qf, kf = fx["q"].astype(np.float32), fx["k"].astype(np.float32)
    if rope:
        qf = oracle_lib.rope(qf, fx["cos"], fx["sin"], round_f16=True)
        kf = oracle_lib.rope(kf, fx["cos"], fx["sin"], round_f16=True)
    out = oracle_lib.attention(qf, kf, fx["v"].astype(np.float32), causal=bool(causal), window=window, nthreads=1)
    assert out.shape == (b, hq, sq, d)
    np.testing.assert_array_equal(out, fx["out"])


@pytest.mark.parametrize("path", I8, ids=[p.stem for p in I8])
def test_i8_fixture_reproduced_by_oracle(oracle_lib, path):
    fx = load(path)
    causal, window, per_token = bool(fx["params"][6]), int(fx["params"][7]), bool(fx["params"][8])
    np.testing.assert_array_equal(oracle_lib.int8_scores(fx["qi"], fx["ki"]), fx["scores"])
    qs = fx["q_scale"] if per_token else float(fx["q_scale"])
    ks = fx["k_scale"] if per_token else float(fx["k_scale"])
    out = oracle_lib.attention_int8(fx["qi"], fx["ki"], fx["vi"], qs, ks, float(fx["v_scale"]),
                                    causal=causal, window=window, nthreads=1)
    np.testing.assert_array_equal(out, fx["out"])


def test_dense_fixture_matches_numpy_softmax():
    fx = load(GOLDEN / "f16_mha_dense_d64.npz")
    q = fx["q"].astype(np.float64)
    k = fx["k"].astype(np.float64)
    v = fx["v"].astype(np.float64)
    s = q @ np.swapaxes(k, -1, -2) / np.sqrt(q.shape[-1])
    p = np.exp(s - s.max(-1, keepdims=True))
    ref = (p / p.sum(-1, keepdims=True)) @ v
    np.testing.assert_allclose(fx["out"], ref, atol=1e-6, rtol=0)


def test_rows_without_keys_fixture_is_zero():
    fx = load(GOLDEN / "f16_rows_without_keys_d64.npz")
    sq, sk = int(fx["params"][3]), int(fx["params"][4])
    assert np.all(fx["out"][:, :, : sq - sk] == 0.0)
    assert np.all(np.abs(fx["out"][:, :, sq - sk:]).sum(-1) > 0)


@pytest.mark.parametrize("path", I8, ids=[p.stem for p in I8])
def test_i8_scores_fixture_matches_numpy(path):
    fx = load(path)
    qi = fx["qi"].astype(np.int64)
    ki = fx["ki"].astype(np.int64)
    ratio = qi.shape[1] // ki.shape[1]
    ref = qi @ np.swapaxes(np.repeat(ki, ratio, axis=1), -1, -2)
    np.testing.assert_array_equal(fx["scores"].astype(np.int64), ref)
