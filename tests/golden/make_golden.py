#!/usr/bin/env python3
"""Write the committed golden data of the quantized matrix-vector path.

The reference ships no vectors for this path (its one test needs a downloaded
model and asserts on text), so the golden data here are made from the seeded
generator and the CPU oracle, and fix both against silent drift:

  synth_digests.json  SHA-256 of every buffer of the five benchmark
                      configurations (Q8_0 2048x2048; the Q4_0 FFN; the Q8_0
                      262144-row LM head; Q4_K 8192x2048 with M = 1/8/32/64
                      activation rows; 128-expert Q4_K MoE with 1 and 16 tokens),
                      as gemma4.kt_amd/synth.py produces them.
  fixtures.npz        small cases of every format: raw GGUF blocks, x, the
                      oracle's restated Vector API output (y), the fp64 dot of the
                      exactly decoded weights (y64) and the tolerance scale
                      sum|w x| per row (ab); plus one MoE case (router logits,
                      routing, Y, Y64, bound).

Run from the repository root: python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "gemma4.kt_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

import synth  # noqa: E402

FORMATS = {"q8_0": 8, "q4_0": 2, "q4_k": 12, "q5_k": 13, "q6_k": 14, "f16": 1, "bf16": 30, "f32": 0}
# rows x cols of each small case: 64-aligned rows, K-quant rows that straddle
# super-blocks (1408), and one row length off the 64-element grid (the scalar tail)
SHAPES = [(8, 512), (4, 1408), (8, 256 + 32)]
FIXTURE_SEED = 0x601D


def config_buffers():
    """(name, buffers) of each benchmark configuration, in a fixed order."""
    yield "q8_0_matvec_2048x2048", synth.q8_0_matvec_2048()
    yield "q4_0_ffn_8192x2048", synth.q4_0_ffn()
    for m in (1, 8, 32, 64):
        yield "q4_k_batched_8192x2048_m%d" % m, synth.q4_k_batched(m)
    yield "q8_0_lm_head_262144x2048", synth.q8_0_lm_head()
    for t in (1, 16):
        yield "moe_q4_k_128x_top8_t%d" % t, synth.moe_q4_k(t)


def digests() -> dict:
    out = {}
    for name, d in config_buffers():
        out[name] = {k: hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest()
                     for k, v in sorted(d.items()) if isinstance(v, np.ndarray)}
    return out


def fixture_arrays(oracle) -> dict:
    arrs = {}
    for fmt, t in FORMATS.items():
        for rows, cols in SHAPES:
            key = "%s_%dx%d" % (fmt, rows, cols)
            raw = synth.weights(FIXTURE_SEED, key, t, rows * cols)  # whole blocks for every shape here
            x = synth.activations(FIXTURE_SEED, key + ".x", cols)
            y = oracle.matmul(t, raw, x, rows, cols)
            y64, ab = oracle.matmul_exact(t, raw, x, rows, cols)
            arrs[key + ".raw"] = raw
            arrs[key + ".x"] = x
            arrs[key + ".y"] = y
            arrs[key + ".y64"] = y64
            arrs[key + ".ab"] = ab
    # one routed MoE case: 6 Q4_K experts, dim 128, ff 64, top-3 of 3 tokens
    E, dim, ff, T, k = 6, 128, 64, 3, 3
    gu = synth.q4_k(FIXTURE_SEED, "moe.gu", E * 2 * ff * dim)
    dn = synth.q4_k(FIXTURE_SEED, "moe.dn", E * dim * ff)
    X = synth.activations(FIXTURE_SEED, "moe.x", T * dim).reshape(T, dim)
    lg = synth.activations(FIXTURE_SEED, "moe.lg", T * E).reshape(T, E)
    ids, w = oracle.route(lg, k, True)
    Y = oracle.moe(12, gu, 12, dn, X, ids, w, dim, ff)
    Y64, B = oracle.moe_exact(12, gu, 12, dn, X, ids, w, dim, ff)
    arrs.update({"moe.gate_up": gu, "moe.down": dn, "moe.x": X, "moe.logits": lg, "moe.ids": ids,
                 "moe.w": w, "moe.y": Y, "moe.y64": Y64, "moe.bound": B,
                 "moe.shape": np.array([E, dim, ff, T, k], np.int32)})
    return arrs


def main() -> None:
    import oracle
    oracle.lib()
    with open(os.path.join(HERE, "synth_digests.json"), "w") as f:
        json.dump(digests(), f, indent=1, sort_keys=True)
        f.write("\n")
    np.savez_compressed(os.path.join(HERE, "fixtures.npz"), **fixture_arrays(oracle))
    print("wrote", os.path.join(HERE, "synth_digests.json"), "and", os.path.join(HERE, "fixtures.npz"))


if __name__ == "__main__":
    main()
