"""Rows whose tolerance scale sum|w_i x_i| is zero or tiny.

The reference forms every weight before its product: Q4_0 as (q - 8) * d
(Q4_0FloatTensor.kt:80-91), Q4_K / Q5_K as fma(q, d*sc, -dmin*m)
(Q4_KFloatTensor.kt:143-148, Q5_KFloatTensor.kt), so a row of weights that are
all exactly zero dots to exactly 0 whatever its scales, and the tolerance
1e-5 * sum|w_i x_i| is 0 there.  The kernels factor the scales out of the block
sums (d * (sum q x - 8 sum x) and d*sc * sum q x - dmin*m * sum x); these tests
check that the factored forms still return exactly 0 on such rows, and stay
inside the tolerance on rows of weights in {-d*sc, 0, d*sc}, on every kernel
variant a row can take: the row engine (one pass, several passes, x read at
use), the multi-token matrix-core kernel and the MoE down projection.

Blocks: Q4_0 with every nibble 8 and d != 0; Q4_K with dmin = 8 d and m = sc,
so w = d*sc*(q - 8); Q5_K with dmin = 16 d and m = sc, w = d*sc*(q - 16).
"""
import numpy as np
import pytest

import synth
from conftest import announce

Q4_0, Q4_K, Q5_K, Q6_K, Q8_0 = 2, 12, 13, 14, 8


def _fp16(v):
    return synth.fp16_bits(np.asarray(v, np.float64))


def _block_kinds(rows, cols, kinds, block):
    """Kind of each block of `block` elements (a block lies inside one row pair:
    kinds come in pairs of rows and 2 * cols is a whole number of blocks)."""
    assert (2 * cols) % block == 0 and all(kinds[r] == kinds[r ^ 1] for r in range(rows - rows % 2))
    return [kinds[(b * block) // cols] for b in range(rows * cols // block)]


def q4_0_rows(rows, cols, kinds, seed=11):
    """kinds[r]: 'zero' (all q = 8), 'pm1' (q in {7, 8, 9}) or 'rand'."""
    rng = np.random.default_rng(seed)
    out = synth.q4_0(seed, "zb", rows * cols).reshape(-1, 18)
    for b, kind in enumerate(_block_kinds(rows, cols, kinds, 32)):
        if kind == "rand":
            continue
        q = np.full(32, 8, np.uint8) if kind == "zero" else rng.integers(7, 10, 32).astype(np.uint8)
        out[b, 2:] = q[:16] | (q[16:] << 4)
    return out.reshape(-1)


def _k_head(rng, dmul):
    d = abs(rng.standard_normal()) * 0.01 + 1e-3
    dh = _fp16([d])
    d16 = float(dh.view(np.float16)[0])
    dmin = _fp16([d16 * dmul])
    assert float(dmin.view(np.float16)[0]) == d16 * dmul  # exact
    sc = rng.integers(1, 64, (1, 8))
    return dh.view(np.uint8), dmin.view(np.uint8), synth.pack_q4k_scales(sc, sc)[0]


def q4_k_rows(rows, cols, kinds, seed=12):
    """Q4_K super-blocks with dmin = 8 d, m = sc: w = d*sc*(q - 8)."""
    rng = np.random.default_rng(seed)
    out = synth.q4_k(seed, "zb", rows * cols).reshape(-1, 144)
    for b, kind in enumerate(_block_kinds(rows, cols, kinds, 256)):
        if kind == "rand":
            continue
        out[b, 0:2], out[b, 2:4], out[b, 4:16] = _k_head(rng, 8.0)
        q = np.full((4, 2, 32), 8, np.uint8) if kind == "zero" else rng.integers(7, 10, (4, 2, 32)).astype(np.uint8)
        out[b, 16:] = (q[:, 0, :] | (q[:, 1, :] << 4)).reshape(128)
    return out.reshape(-1)


def q5_k_rows(rows, cols, kinds, seed=13):
    """Q5_K super-blocks with dmin = 16 d, m = sc: w = d*sc*(q - 16)."""
    rng = np.random.default_rng(seed)
    out = synth.q5_k(seed, "zb", rows * cols).reshape(-1, 176)
    for b, kind in enumerate(_block_kinds(rows, cols, kinds, 256)):
        if kind == "rand":
            continue
        out[b, 0:2], out[b, 2:4], out[b, 4:16] = _k_head(rng, 16.0)
        # q[g, h, l] in 15..17 (or all 16): nibble q & 15, fifth bit q >> 4 in bit 2g + h of qh[l]
        q = np.full((4, 2, 32), 16, np.uint8) if kind == "zero" else \
            rng.integers(15, 18, (4, 2, 32)).astype(np.uint8)
        nib, hb = q & 15, q >> 4
        out[b, 48:] = (nib[:, 0, :] | (nib[:, 1, :] << 4)).reshape(128)
        qh = np.zeros(32, np.uint8)
        for g in range(4):
            for h in range(2):
                qh |= (hb[g, h, :] << (2 * g + h)).astype(np.uint8)
        out[b, 16:48] = qh
    return out.reshape(-1)


BUILD = {Q4_0: q4_0_rows, Q4_K: q4_k_rows, Q5_K: q5_k_rows}


def _kinds(rows):
    return [("zero", "pm1", "rand")[(r // 2) % 3] for r in range(rows)]


def _check(y, y64, ab, kinds, what):
    y = np.asarray(y, np.float64)
    zero = np.array([k == "zero" for k in kinds])
    assert np.all(ab[zero] == 0.0) and np.all(y64[zero] == 0.0)
    bad = np.nonzero(y[zero] != 0.0)[0]
    assert bad.size == 0, "%s: rows of zero weights gave %r" % (what, y[zero][bad[:4]])
    err = np.abs(y - y64)
    assert np.all(err <= 1e-5 * ab), "%s: max err/bound %g" % (what, float(np.max(err / np.maximum(ab, 1e-300))))


# ---------------------------------------------------------------- CPU pins ---

@pytest.mark.parametrize("t", [Q4_0, Q4_K, Q5_K])
def test_reference_gives_exact_zero_on_zero_rows(oracle, t):
    """The restated reference (weights formed first) returns exactly 0 on the
    zero rows, and the blocks decode as intended: w in {0} or {-d*sc, 0, d*sc}."""
    rows, cols = 12, 1024
    kinds = _kinds(rows)
    raw = BUILD[t](rows, cols, kinds)
    x = synth.activations(5, "x", cols)
    w = oracle.dequant(t, raw, 0, rows * cols).reshape(rows, cols)
    for r, k in enumerate(kinds):
        if k == "zero":
            assert np.all(w[r] == 0.0)
        elif k == "pm1":
            # per 32-weight sub-block the magnitudes are 0 and one scale
            for blk in np.abs(w[r]).reshape(-1, 32):
                assert len(set(blk.tolist()) - {0.0}) <= 1
            assert np.any(w[r] > 0) and np.any(w[r] < 0) and np.any(w[r] == 0)
    for mode in (oracle.MODE_VECTOR, oracle.MODE_SCALAR):
        y = oracle.matmul(t, raw, x, rows, cols, mode=mode)
        y64, ab = oracle.matmul_exact(t, raw, x, rows, cols)
        _check(y, y64, ab, kinds, "oracle mode %d" % mode)


# ------------------------------------------------------------------ GPU ---

@pytest.mark.gpu
@pytest.mark.parametrize("t", [Q4_0, Q4_K, Q5_K])
@pytest.mark.parametrize("rows,cols", [(96, 2048), (48, 1408), (24, 16384), (30, 512)])
def test_zero_rows_matvec(g4, ctx, oracle, t, rows, cols):
    """One pass (2048), x read at use (1408 = 22 chunks), several column passes
    (16384), 16-lane rows (512)."""
    announce("zero-bound matvec type %d %dx%d" % (t, rows, cols))
    kinds = _kinds(rows)
    raw = BUILD[t](rows, cols, kinds)
    x = synth.activations(6, "x%d" % cols, cols)
    w = g4.FloatTensorFactory.create(ctx, t, raw, rows * cols)
    y = np.empty(rows, np.float32)
    w.matmul(x, y, rows, cols)
    y64, ab = oracle.matmul_exact(t, raw, x, rows, cols)
    _check(y, y64, ab, kinds, "matvec")
    w.free()


@pytest.mark.gpu
@pytest.mark.parametrize("t,m,rows", [(Q4_K, 2, 96), (Q4_K, 8, 96), (Q4_K, 33, 96), (Q4_0, 4, 96), (Q5_K, 3, 96),
                                      (Q4_K, 200, 1280)])
def test_zero_rows_batched(g4, ctx, oracle, t, m, rows):
    """Several activation rows: the matrix-core kernel for Q4_K (16(q - 8)
    operands; with 200 tokens over 1280 rows, five row tiles per workgroup, the
    16 q operands less sum(128 x), whose difference is exactly 0 for q = 8), the
    row engine per token otherwise."""
    announce("zero-bound batched type %d M=%d rows=%d" % (t, m, rows))
    cols = 2048
    kinds = _kinds(rows)
    raw = BUILD[t](rows, cols, kinds)
    X = synth.activations(7, "X%d" % m, m * cols).reshape(m, cols)
    w = g4.FloatTensorFactory.create(ctx, t, raw, rows * cols)
    Y = w.matmul_batch(X, rows, cols)
    for i in range(m):
        y64, ab = oracle.matmul_exact(t, raw, X[i], rows, cols)
        _check(Y[i], y64, ab, kinds, "batched token %d" % i)
    w.free()


@pytest.mark.gpu
def test_zero_down_experts_give_exact_zero(g4, ctx, oracle):
    """MoE whose down slabs hold only zero weights: every output is exactly 0
    (the reference's down matmul returns 0 rows, saxpy adds 0 * w)."""
    announce("zero-bound moe down")
    E, dim, ff, T, k = 8, 256, 1408, 3, 4
    gu = synth.q4_k(14, "gu", E * 2 * ff * dim)
    dn = q4_k_rows(E * dim, ff, ["zero"] * (E * dim))  # every down weight exactly 0
    X = synth.activations(14, "x", T * dim).reshape(T, dim)
    logits = synth.activations(14, "lg", T * E).reshape(T, E)
    wgu = g4.FloatTensorFactory.create(ctx, Q4_K, gu, E * 2 * ff * dim)
    wdn = g4.FloatTensorFactory.create(ctx, Q4_K, dn, E * dim * ff)
    Y, ids, wts = g4.moe_routed(ctx, wgu, wdn, X, logits, k, True, dim, ff)
    assert np.all(Y == 0.0)
    Y2 = g4.moe(ctx, wgu, wdn, X, ids, wts, dim, ff)
    assert np.all(Y2 == 0.0)
    wgu.free()
    wdn.free()
