"""Committed golden data (tests/golden/, written by tests/golden/make_golden.py).

CPU checks: the seeded generator still produces the benchmark buffers whose
SHA-256 digests are committed, and the oracle still reproduces the committed
small fixtures bit for bit (restated Vector API outputs, fp64 exact dots,
routing and MoE), with the fp64 values also re-derived from the independent
numpy decode.  The GPU side of the same fixtures is in test_gpu_golden.py."""
import hashlib
import json
import os
import sys

import numpy as np
import pytest

import npref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_fixtures() -> dict:
    with np.load(os.path.join(GOLDEN, "fixtures.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def dot_cases(fx: dict):
    """(key, ggml type, rows, cols) of every matvec fixture."""
    types = {"q8_0": 8, "q4_0": 2, "q4_k": 12, "q5_k": 13, "q6_k": 14, "f16": 1, "bf16": 30, "f32": 0}
    for k in sorted(fx):
        if k.endswith(".raw") and not k.startswith("moe."):
            key = k[:-4]
            fmt, shape = key.rsplit("_", 1)
            rows, cols = (int(v) for v in shape.split("x"))
            yield key, types[fmt], rows, cols


def same_bits(a, b) -> bool:
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


def test_synth_digests_unchanged():
    if GOLDEN not in sys.path:
        sys.path.insert(0, GOLDEN)
    import make_golden
    want = json.load(open(os.path.join(GOLDEN, "synth_digests.json")))
    got = {}
    for name, d in make_golden.config_buffers():
        got[name] = {k: hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest()
                     for k, v in sorted(d.items()) if isinstance(v, np.ndarray)}
        assert got[name] == want[name], name
    assert set(got) == set(want)


def test_fixture_cases_cover_every_format():
    fx = load_fixtures()
    cases = list(dot_cases(fx))
    assert {t for _, t, _, _ in cases} == {8, 2, 12, 13, 14, 1, 30, 0}
    assert len(cases) == 8 * 3


def test_oracle_reproduces_fixtures(oracle):
    fx = load_fixtures()
    for key, t, rows, cols in dot_cases(fx):
        raw, x = fx[key + ".raw"], fx[key + ".x"]
        assert same_bits(oracle.matmul(t, raw, x, rows, cols), fx[key + ".y"]), key
        y64, ab = oracle.matmul_exact(t, raw, x, rows, cols)
        assert same_bits(y64, fx[key + ".y64"]) and same_bits(ab, fx[key + ".ab"]), key
        # the fp64 values from the independent numpy decode of the same bytes
        w = npref.dequant(t, raw).astype(np.float64).reshape(rows, cols)
        xd = x.astype(np.float64)
        assert np.all(np.abs(w @ xd - fx[key + ".y64"]) <= 1e-12 * (np.abs(w) @ np.abs(xd))), key
        assert np.allclose(np.abs(w) @ np.abs(xd), fx[key + ".ab"], rtol=1e-12, atol=0), key
        # and the restated reference output sits inside the tolerance
        assert np.all(np.abs(fx[key + ".y"] - fx[key + ".y64"]) <= 1e-5 * fx[key + ".ab"]), key


def test_oracle_reproduces_moe_fixture(oracle):
    fx = load_fixtures()
    E, dim, ff, T, k = (int(v) for v in fx["moe.shape"])
    ids, w = oracle.route(fx["moe.logits"], k, True)
    assert same_bits(ids, fx["moe.ids"]) and same_bits(w, fx["moe.w"])
    Y = oracle.moe(12, fx["moe.gate_up"], 12, fx["moe.down"], fx["moe.x"], ids, w, dim, ff)
    assert same_bits(Y, fx["moe.y"])
    Y64, B = oracle.moe_exact(12, fx["moe.gate_up"], 12, fx["moe.down"], fx["moe.x"], ids, w, dim, ff)
    assert np.allclose(Y64, fx["moe.y64"], rtol=1e-13, atol=0) and np.allclose(B, fx["moe.bound"], rtol=1e-13)
    assert fx["moe.gate_up"].size == E * 2 * ff * dim // 256 * 144


@pytest.mark.parametrize("mutation", ["flip_weight_byte", "perturb_x"])
def test_fixture_check_catches_a_change(oracle, mutation):
    # a changed byte of the weights or a changed activation moves the oracle off the fixture
    fx = load_fixtures()
    key, t, rows, cols = [c for c in dot_cases(fx) if c[0] == "q4_k_4x1408"][0]
    raw, x = fx[key + ".raw"].copy(), fx[key + ".x"].copy()
    if mutation == "flip_weight_byte":
        raw[200] ^= 0x11
    else:
        x[5] = np.float32(x[5] * 1.001)
    assert not same_bits(oracle.matmul(t, raw, x, rows, cols), fx[key + ".y"])
