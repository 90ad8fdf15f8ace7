"""Pins of the CPU oracle (oracle/g4_oracle.c) against what the mathematics and
independent implementations fix.  The reference ships no golden vectors for this
path, so each oracle function is checked against:
  * numpy / torch conversions over every 16-bit pattern (fp16, bf16);
  * a second, independent numpy restatement of the block layouts (tests/npref.py)
    and hand-derived known answers;
  * fp64 brute force for every dot product;
  * closed-form special cases (argmax ties/NaN, softmax, top-k, gelu).
Mutation checks at the end show the comparisons catch the plausible mistakes
(nibble order, scale/min swap, dropped head/tail)."""
import numpy as np
import pytest
import torch

import npref
import synth

Q8_0, Q4_0, Q4_K, Q5_K, Q6_K, F16, BF16, F32 = 8, 2, 12, 13, 14, 1, 30, 0
ALL = [Q8_0, Q4_0, Q4_K, Q5_K, Q6_K, F16, BF16, F32]


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn]))


# ---------------------------------------------------------- 16-bit floats ---

def test_fp16_decode_all_patterns(oracle):
    h = np.arange(65536, dtype=np.uint32)
    ours = oracle.fp16_to_f32_array(h)
    ref = h.astype(np.uint16).view(np.float16).astype(np.float32)
    assert same_bits(ours, ref)
    # payload of NaNs kept exactly (Float.float16ToFloat keeps the significand bits)
    nan = (h >> 10 & 0x1F) == 0x1F
    nan &= (h & 0x3FF) != 0
    assert np.array_equal(ours.view(np.uint32)[nan] & 0x7FFFFF, (h[nan] & 0x3FF) << 13)


def test_fp16_vector_decode_closed_form(oracle):
    # F16FloatTensor.kt:59-61: exponent 0 -> signed zero, exponent 31 -> 2^16 * (1 + m/1024), else IEEE.
    h = np.arange(65536, dtype=np.uint32)
    ours = oracle.fp16_vec_decode_array(h)
    e, m, s = (h >> 10) & 0x1F, h & 0x3FF, (h >> 15) & 1
    sign = np.where(s == 1, -1.0, 1.0)
    expect = np.where(e == 0, sign * 0.0,
                      np.where(e == 31, sign * np.ldexp(1.0 + m / 1024.0, 16),
                               h.astype(np.uint16).view(np.float16).astype(np.float64))).astype(np.float32)
    assert same_bits(ours, expect)
    assert np.array_equal(np.signbit(ours), s == 1)


def test_bf16_decode_all_patterns(oracle):
    h = np.arange(65536, dtype=np.int64)
    ours = oracle.dequant(BF16, h.astype(np.uint16), 0, 65536)
    ref = torch.from_numpy(h.astype(np.uint16).view(np.int16)).view(torch.bfloat16).float().numpy()
    assert same_bits(ours, ref)


# ------------------------------------------------------------- dequant ---

def _random_blocks(t, n_elems, seed=7):
    return synth.weights(seed, "pin%d" % t, t, n_elems)


@pytest.mark.parametrize("t", ALL)
def test_dequant_matches_numpy_restatement(oracle, t):
    n = 256 * 40
    raw = _random_blocks(t, n)
    assert same_bits(oracle.dequant(t, raw, 0, n), npref.dequant(t, raw))
    # get() at arbitrary indices equals the bulk decode
    idx = np.random.default_rng(3).integers(0, n, 200)
    assert same_bits([oracle.get(t, raw, int(i)) for i in idx], npref.dequant(t, raw)[idx])


def test_q8_0_known_values(oracle):
    # d = 0.5 (0x3800), q = -127..127 sampled: w = q * d exactly
    q = np.array(list(range(-127, -111)) + list(range(112, 128)), dtype=np.int8)
    blk = np.concatenate([np.array([0x00, 0x38], np.uint8), q.view(np.uint8)])
    assert same_bits(oracle.dequant(Q8_0, blk, 0, 32), q.astype(np.float32) * 0.5)


def test_q4_0_known_values(oracle):
    # low nibbles 0..15 -> elements 0..15, high nibbles 15..0 -> elements 16..31; d = 2.0 (0x4000)
    qs = np.array([(i & 0xF) | ((15 - i) << 4) for i in range(16)], np.uint8)
    blk = np.concatenate([np.array([0x00, 0x40], np.uint8), qs])
    expect = np.array([(i - 8) * 2.0 for i in range(16)] + [((15 - i) - 8) * 2.0 for i in range(16)], np.float32)
    assert same_bits(oracle.dequant(Q4_0, blk, 0, 32), expect)


# hand-derived from the 12-byte layout (bytes 0..3: sc0..3 low 6 bits, top 2 bits
# = sc4..7 >> 4; bytes 4..7: m0..3 and top bits of m4..7; bytes 8..11: sc4..7 low
# nibble | m4..7 low nibble << 4)
Q4K_SCALES_KAT = np.array([0xC1, 0x02, 0x43, 0x84, 0x05, 0xC6, 0x07, 0x48, 0x21, 0x43, 0x65, 0x87], np.uint8)
Q4K_SC_KAT = [1, 2, 3, 4, 49, 3, 21, 39]
Q4K_M_KAT = [5, 6, 7, 8, 2, 52, 6, 24]


def test_q4k_scale_min_known_answer(oracle):
    assert [oracle.q4k_scale_min(j, Q4K_SCALES_KAT, False) for j in range(8)] == Q4K_SC_KAT
    assert [oracle.q4k_scale_min(j, Q4K_SCALES_KAT, True) for j in range(8)] == Q4K_M_KAT


def test_q4k_scale_min_roundtrip_all_pairs(oracle):
    # every (sc, m) value in every one of the 8 positions, packed by the quantizer direction
    rng = np.random.default_rng(11)
    for rep in range(64):
        sc = rng.integers(0, 64, (1, 8))
        m = rng.integers(0, 64, (1, 8))
        sc[0, rep % 8] = rep  # sweep 0..63 through each slot
        m[0, (rep + 3) % 8] = 63 - rep
        packed = npref.pack_q4k_scales_quantizer(sc, m)[0]
        assert [oracle.q4k_scale_min(j, packed, False) for j in range(8)] == list(sc[0])
        assert [oracle.q4k_scale_min(j, packed, True) for j in range(8)] == list(m[0])
    # the synthetic generator's packer writes the same bytes
    sc = rng.integers(0, 64, (50, 8))
    m = rng.integers(0, 64, (50, 8))
    assert np.array_equal(synth.pack_q4k_scales(sc, m), npref.pack_q4k_scales_quantizer(sc, m))


def _q4k_block(d, dmin, sc, m, q):
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([d], np.float16).view(np.uint8)
    blk[2:4] = np.array([dmin], np.float16).view(np.uint8)
    blk[4:16] = npref.pack_q4k_scales_quantizer(np.array([sc]), np.array([m]))[0]
    q = np.asarray(q).reshape(4, 2, 32)
    blk[16:] = (q[:, 0, :] | (q[:, 1, :] << 4)).reshape(-1).astype(np.uint8)
    return blk


@pytest.mark.parametrize("case", ["extremes", "zero_d", "subnormal_d", "random"])
def test_q4k_known_values(oracle, case):
    rng = np.random.default_rng(5)
    if case == "extremes":
        d, dmin, sc, m = 0.0625, 0.125, [0, 63, 0, 63, 63, 0, 63, 0], [63, 0, 63, 0, 0, 63, 0, 63]
        q = np.tile(np.array([0, 15] * 16), 8)
    elif case == "zero_d":
        d, dmin, sc, m = 0.0, 0.25, list(range(8)), list(range(60, 68 - 0))[:8]
        m = [60, 61, 62, 63, 1, 2, 3, 4]
        q = rng.integers(0, 16, 256)
    elif case == "subnormal_d":
        d, dmin, sc, m = 2.0 ** -20, 2.0 ** -22, [63] * 8, [1] * 8
        q = rng.integers(0, 16, 256)
    else:
        d, dmin = 0.0123, 0.0071
        sc, m = list(rng.integers(0, 64, 8)), list(rng.integers(0, 64, 8))
        q = rng.integers(0, 16, 256)
    blk = _q4k_block(d, dmin, sc, m, q)
    d32 = np.float32(np.float16(d))
    dm32 = np.float32(np.float16(dmin))
    sub = np.repeat(np.arange(8), 32)
    expect = (np.float32(d32) * np.array(sc, np.float32)[sub]) * np.asarray(q, np.float32) - \
        (np.float32(dm32) * np.array(m, np.float32)[sub])
    assert same_bits(oracle.dequant(Q4_K, blk, 0, 256), expect.astype(np.float32))


def _q5k_block(d, dmin, sc, m, q5):
    """Pack a Q5_K super-block from 256 five-bit values (weight e of group g,
    half h = (e % 64) // 32, lane l: nibble in qs[32g + l], 5th bit in bit 2g + h of qh[l])."""
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.array([d], np.float16).view(np.uint8)
    blk[2:4] = np.array([dmin], np.float16).view(np.uint8)
    blk[4:16] = npref.pack_q4k_scales_quantizer(np.array([sc]), np.array([m]))[0]
    q5 = np.asarray(q5, np.int64)
    for e in range(256):
        g, h, l = e // 64, (e % 64) // 32, e % 32
        blk[48 + 32 * g + l] |= (q5[e] & 15) << (4 * h)
        blk[16 + l] |= (q5[e] >> 4) << (2 * g + h)
    return blk


@pytest.mark.parametrize("case", ["extremes", "all_high_bits", "random"])
def test_q5k_known_values(oracle, case):
    rng = np.random.default_rng(6)
    if case == "extremes":
        d, dmin, sc, m = 0.0625, 0.125, [0, 63, 0, 63, 63, 0, 63, 0], [63, 0, 63, 0, 0, 63, 0, 63]
        q5 = np.tile(np.array([0, 31, 16, 15]), 64)
    elif case == "all_high_bits":
        d, dmin, sc, m = 0.5, 0.25, [1, 2, 3, 4, 5, 6, 7, 8], [8, 7, 6, 5, 4, 3, 2, 1]
        q5 = 16 + rng.integers(0, 16, 256)
    else:
        d, dmin = 0.0123, 0.0071
        sc, m = list(rng.integers(0, 64, 8)), list(rng.integers(0, 64, 8))
        q5 = rng.integers(0, 32, 256)
    blk = _q5k_block(d, dmin, sc, m, q5)
    d32, dm32 = np.float32(np.float16(d)), np.float32(np.float16(dmin))
    sub = np.repeat(np.arange(8), 32)
    expect = (d32 * np.array(sc, np.float32)[sub]) * np.asarray(q5, np.float32) - \
        (dm32 * np.array(m, np.float32)[sub])
    assert same_bits(oracle.dequant(Q5_K, blk, 0, 256), expect.astype(np.float32))
    assert same_bits(npref.dequant(Q5_K, blk), expect.astype(np.float32))


def _q6k_block(d, scales, q6):
    """Pack a Q6_K super-block from 256 values in -32..31 (weight e: half n = e // 128,
    row r = (e % 128) // 32, lane l = e % 32; low nibble in ql[64n + l + 32 (r & 1)]
    at shift 4 (r >> 1), bit pair at shift 2r of qh[32n + l])."""
    blk = np.zeros(210, np.uint8)
    v = np.asarray(q6, np.int64) + 32
    for e in range(256):
        n, r, l = e // 128, (e % 128) // 32, e % 32
        blk[64 * n + l + 32 * (r & 1)] |= (v[e] & 15) << (4 * (r >> 1))
        blk[128 + 32 * n + l] |= (v[e] >> 4) << (2 * r)
    blk[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    blk[208:210] = np.array([d], np.float16).view(np.uint8)
    return blk


@pytest.mark.parametrize("case", ["extremes", "negative_scales", "random"])
def test_q6k_known_values(oracle, case):
    rng = np.random.default_rng(9)
    if case == "extremes":
        d, scales = 0.5, [127, -128, 1, -1, 0, 64, -64, 2] * 2
        q6 = np.tile(np.array([-32, 31, 0, -1]), 64)
    elif case == "negative_scales":
        d, scales = 2.0 ** -10, list(-np.arange(1, 17) * 8)
        q6 = rng.integers(-32, 32, 256)
    else:
        d, scales = 0.0123, list(rng.integers(-128, 128, 16))
        q6 = rng.integers(-32, 32, 256)
    blk = _q6k_block(d, scales, q6)
    d32 = np.float32(np.float16(d))
    sidx = (np.arange(256) // 128) * 8 + ((np.arange(256) % 128) // 32) * 2 + (np.arange(256) % 32) // 16
    expect = (d32 * np.array(scales, np.float32)[sidx]) * np.asarray(q6, np.float32)
    assert same_bits(oracle.dequant(Q6_K, blk, 0, 256), expect.astype(np.float32))
    assert same_bits(npref.dequant(Q6_K, blk), expect.astype(np.float32))


# ----------------------------------------------------------------- dots ---

def _offsets(t):
    bs = {Q8_0: 32, Q4_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}.get(t, 1)
    # aligned rows, unaligned heads and tails, shorter than one block, odd sizes
    return [(0, 2048), (bs, 1024), (7, 900), (max(bs - 3, 1), 5), (3, bs + 9), (0, 17), (64, 1408)]


@pytest.mark.parametrize("t", ALL)
def test_exact_dot_matches_numpy_fp64(oracle, t):
    n = 256 * 24
    raw = _random_blocks(t, n, seed=21)
    x = synth.activations(21, "x", n)
    w = npref.dequant(t, raw).astype(np.float64)
    for off, size in _offsets(t):
        v, a = oracle.exact_dot(t, raw, off, x, size)
        ref = float(np.dot(w[off:off + size], x[:size].astype(np.float64)))
        refa = float(np.sum(np.abs(w[off:off + size] * x[:size])))
        assert abs(v - ref) <= 1e-12 * max(refa, 1e-300)
        assert abs(a - refa) <= 1e-12 * max(refa, 1e-300)


@pytest.mark.parametrize("t", ALL)
@pytest.mark.parametrize("mode", [0, 1])
def test_reference_dots_within_tolerance(oracle, t, mode):
    """The restated vectorDot (mode 0) and scalarDot (mode 1) are within the
    accumulation-order tolerance 1e-5 * sum|w x| of the exact dot."""
    n = 256 * 24
    raw = _random_blocks(t, n, seed=22)
    x = synth.activations(22, "x", n)
    for off, size in _offsets(t):
        v = oracle.vector_dot(t, raw, off, x, size) if mode == 0 else oracle.scalar_dot(t, raw, off, x, size)
        ex, a = oracle.exact_dot(t, raw, off, x, size)
        assert abs(v - ex) <= 1e-5 * a + 1e-30, (off, size, v, ex, a)


def test_vector_dot_f16_uses_vector_decode_then_exact_tail(oracle):
    # a subnormal fp16 weight is flushed inside loopBound(size) and kept in the tail
    w = np.zeros(20, np.uint16)
    w[3] = 0x0001   # 2^-24, inside the first 16 lanes
    w[18] = 0x0001  # in the scalar tail (size 20 -> loopBound 16)
    x = np.full(20, 2.0 ** 20, np.float32)
    v = oracle.vector_dot(F16, w.view(np.uint8), 0, x, 20)
    assert v == np.float32(2.0 ** -24 * 2.0 ** 20)  # only the tail element counts


def test_matmul_rows_and_offset(oracle):
    n_rows, dim1 = 12, 512
    raw = _random_blocks(Q4_K, 40 * 256, seed=23)
    x = synth.activations(23, "x", dim1)
    off = 3 * 256
    out = oracle.matmul(Q4_K, raw, x, n_rows, dim1, this_offset=off, threads=2)
    for i in range(n_rows):
        assert out[i] == np.float32(oracle.vector_dot(Q4_K, raw, off + i * dim1, x, dim1))


# -------------------------------------------------------- argmax / route ---

def test_argmax_semantics(oracle):
    assert oracle.argmax(np.array([1, 3, 3, 2], np.float32)) == 1              # first of ties
    assert oracle.argmax(np.array([-0.0, 0.0], np.float32)) == 0                # -0 == +0
    assert oracle.argmax(np.array([np.nan, 5, 6], np.float32)) == 0             # NaN first wins
    assert oracle.argmax(np.array([1, np.nan, 0.5], np.float32)) == 0           # NaN never wins
    assert oracle.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    assert oracle.argmax(np.array([-np.inf, np.inf, np.inf], np.float32)) == 1
    v = synth.activations(9, "am", 10000)
    assert oracle.argmax(v) == int(np.argmax(v))
    assert oracle.argmax(v, 100, 500) == 100 + int(np.argmax(v[100:600]))


def test_softmax_matches_fp64(oracle):
    v = synth.activations(10, "sm", 128)
    p = oracle.softmax(v)
    e = np.exp(v.astype(np.float64) - v.max())
    ref = e / e.sum()
    assert np.max(np.abs(p - ref)) <= 1e-6 * ref.max()
    assert abs(float(np.sum(p.astype(np.float64))) - 1.0) < 1e-5


def test_topk_order_and_ties(oracle):
    p = np.array([0.1, 0.3, 0.3, 0.05, 0.25], np.float32)
    idx, val, masked = oracle.topk(p, 3)
    assert list(idx) == [1, 2, 4] and list(val) == [np.float32(0.3), np.float32(0.3), np.float32(0.25)]
    assert np.isneginf(masked[[1, 2, 4]]).all()
    # more than available: remaining scans see only -inf and keep index 0
    idx, val, _ = oracle.topk(np.array([0.5, 0.5], np.float32), 3)
    assert list(idx) == [0, 1, 0] and np.isneginf(val[2])
    rng = np.random.default_rng(1)
    for _ in range(20):
        v = rng.standard_normal(128).astype(np.float32)
        idx, _, _ = oracle.topk(v, 8)
        assert list(idx) == list(np.argsort(-v, kind="stable")[:8])


def test_route_renormalised_and_scaled(oracle):
    lg = synth.activations(12, "rt", 4 * 128).reshape(4, 128)
    ids, w = oracle.route(lg, 8, True)
    ids0, w0 = oracle.route(lg, 8, False)
    assert np.array_equal(ids, ids0)
    for t in range(4):
        p = oracle.softmax(lg[t])
        assert list(ids[t]) == list(np.argsort(-p, kind="stable")[:8])
        assert np.array_equal(w0[t], p[ids[t]])
        assert abs(float(w[t].astype(np.float64).sum()) - 1.0) < 1e-6
    scale = np.linspace(0.5, 2.0, 128).astype(np.float32)
    ids2, w2 = oracle.route(lg, 8, False, scale)
    assert np.array_equal(w2, w0 * scale[ids0])


def test_gelu_matches_torch_tanh_form(oracle):
    xs = np.linspace(-8, 8, 1001).astype(np.float32)
    ours = np.array([oracle.gelu(float(v)) for v in xs], np.float32)
    ref = torch.nn.functional.gelu(torch.from_numpy(xs.astype(np.float64)), approximate="tanh").numpy()
    # 1 + tanh cancels for x << 0 in double in both forms; compare relative plus a tiny absolute floor
    assert np.all(np.abs(ours - ref) <= 2e-7 * np.abs(ref) + 1e-12)


def test_tanh_is_fdlibms_within_an_ulp(oracle):
    """or_tanh follows fdlibm's tanh steps (StrictMath.tanh's algorithm) over the C
    library's expm1, so its bit parity with the JVM's tanh is unpinned.
    Pinned against mpmath at 60 digits: within 2 ulps everywhere (Math.tanh's
    contract allows 2.5), odd, and the special values; near -1 (where gelu's
    1 + tanh keeps only the low bits) it is the correctly rounded double."""
    mpmath = pytest.importorskip("mpmath")
    mpmath.mp.dps = 60
    rng = np.random.default_rng(62)
    xs = np.concatenate([10.0 ** rng.uniform(-20, np.log10(30.0), 3000), np.linspace(0.0, 25.0, 501),
                         [2.0 ** -55, np.nextafter(2.0 ** -55, 0), 1.0, np.nextafter(1.0, 0), 22.0,
                          np.nextafter(22.0, 0)]])
    for x in xs:
        x = float(x)
        got = oracle.tanh(x)
        exact = mpmath.tanh(mpmath.mpf(x))
        ulp = np.spacing(abs(float(exact))) if exact != 0 else 5e-324
        assert abs(mpmath.mpf(got) - exact) <= 2 * ulp, x
        assert oracle.tanh(-x) == -got
    cr = 0
    for z in np.linspace(2.0, 8.0, 2001):
        cr += oracle.tanh(-float(z)) == float(mpmath.tanh(mpmath.mpf(-float(z))))
    assert cr >= 1990
    assert oracle.tanh(np.inf) == 1.0 and oracle.tanh(-np.inf) == -1.0 and np.isnan(oracle.tanh(np.nan))
    assert oracle.tanh(30.0) == 1.0 and oracle.tanh(1e-300) == 1e-300
    assert np.signbit(oracle.tanh(-0.0)) and oracle.tanh(-0.0) == 0.0


# ---------------------------------------------------------------- mutations ---
# The comparisons above must fail for plausible mistakes; plant each mistake in a
# copy of the numpy restatement and check the oracle disagrees with it.

def test_mutation_nibble_order_detected(oracle):
    raw = _random_blocks(Q4_0, 32 * 64, seed=31)
    blk = raw.reshape(-1, 18)
    d = npref._f16(blk[:, 0:2])
    swapped = np.concatenate([blk[:, 2:] >> 4, blk[:, 2:] & 0xF], axis=1).astype(np.float32) - 8
    wrong = (swapped * d[:, None]).reshape(-1)
    assert not same_bits(oracle.dequant(Q4_0, raw, 0, 32 * 64), wrong)


def test_mutation_scale_min_swap_detected(oracle):
    raw = _random_blocks(Q4_K, 256 * 8, seed=32)
    sb = raw.reshape(-1, 144).copy()
    sc, m = npref.q4k_unpack_scales(sb[:, 4:16])
    sb[:, 4:16] = npref.pack_q4k_scales_quantizer(m, sc)  # scales and mins exchanged
    assert not same_bits(oracle.dequant(Q4_K, raw, 0, 256 * 8), npref.dequant(Q4_K, sb.reshape(-1)))


def test_mutation_dropped_tail_detected(oracle):
    raw = _random_blocks(Q8_0, 32 * 8, seed=33)
    x = synth.activations(33, "x", 256)
    ex, a = oracle.exact_dot(Q8_0, raw, 7, x, 200)
    dropped, _ = oracle.exact_dot(Q8_0, raw, 7, x, 192)
    assert abs(dropped - ex) > 1e-5 * a


# ---------------------------------------------------------- decode step ---
# rmsnorm (Llama.kt:27-78), soft-capping (Llama.kt:403-406) and the blocks built
# from them.  Pins: fp64 brute force with eps large enough to matter, closed forms
# (constant vectors, unit mean square), exact power-of-two scale invariance, the
# forms' product order on inputs whose sum of squares is exact, and the blocks
# as compositions of the individually pinned functions.

def _norm_inputs(n, seed=7):
    rng = np.random.default_rng(seed)
    return rng.standard_normal(n).astype(np.float32), (1 + 0.25 * rng.standard_normal(n)).astype(np.float32)


@pytest.mark.parametrize("eps", [1e-6, 0.1])
@pytest.mark.parametrize("n", [1, 7, 256, 2048])
def test_rmsnorm_vs_fp64(oracle, n, eps):
    x, w = _norm_inputs(n)
    exact = oracle.rmsnorm_exact(x, w, eps)
    for form in (oracle.NORM_WEIGHT_AFTER, oracle.NORM_WEIGHT_FIRST):
        got = oracle.rmsnorm(x, w, eps, form).astype(np.float64)
        assert np.all(np.abs(got - exact) <= 1e-6 * np.abs(exact) + 1e-30), form
    got = oracle.rmsnorm(x, None, eps, oracle.NORM_NO_WEIGHT).astype(np.float64)
    ex = oracle.rmsnorm_exact(x, None, eps)
    assert np.all(np.abs(got - ex) <= 1e-6 * np.abs(ex))
    # eps sits inside the root, after the mean: moving it changes the result well past 1e-6
    ss = float(np.sum(x.astype(np.float64) ** 2))
    wrong = w * x / np.sqrt((ss + eps) / n)
    assert n == 1 or eps < 0.01 or np.max(np.abs(wrong - exact) / np.abs(exact)) > 1e-3


def test_rmsnorm_closed_forms(oracle):
    # constant vector a: s = 1/sqrt(a^2 + eps) (the mean of equal squares is exact)
    for a, eps in [(3.0, 0.0), (0.5, 1e-6), (1e-3, 1e-6)]:
        x = np.full(64, a, np.float32)
        got = oracle.rmsnorm(x, None, eps, oracle.NORM_NO_WEIGHT)
        assert np.allclose(got, a / np.sqrt(np.float64(a) ** 2 + np.float64(np.float32(eps))), rtol=2e-7, atol=0)
    # unit mean square without eps and weight
    x, _ = _norm_inputs(2048, seed=3)
    out = oracle.rmsnorm(x, None, 0.0, oracle.NORM_NO_WEIGHT).astype(np.float64)
    assert abs(np.mean(out ** 2) - 1.0) < 1e-6
    # scaling x by 2 scales ss by 4 and s by 1/2 exactly (eps = 0): same bits
    w = _norm_inputs(2048, seed=4)[1]
    assert same_bits(oracle.rmsnorm(2 * x, w, 0.0), oracle.rmsnorm(x, w, 0.0))


def test_rmsnorm_form_order(oracle):
    # integer x: every partial sum of squares is exact, so s is fixed and the
    # forms differ only in the product order, which these inputs expose
    rng = np.random.default_rng(11)
    x = rng.integers(-64, 65, 2048).astype(np.float32)
    w = (1 + 0.25 * rng.standard_normal(2048)).astype(np.float32)
    ss = np.float32(np.sum(x.astype(np.float64) ** 2))  # exact: < 2^24
    assert float(ss) == float(np.sum(x.astype(np.float64) ** 2))
    s = np.float32(1.0 / np.sqrt(np.float64(np.float32(ss / np.float32(2048)) + np.float32(1e-6))))
    after = oracle.rmsnorm(x, w, 1e-6, oracle.NORM_WEIGHT_AFTER)
    first = oracle.rmsnorm(x, w, 1e-6, oracle.NORM_WEIGHT_FIRST)
    assert same_bits(after, w * (s * x))
    assert same_bits(first, (w * s) * x)
    assert not same_bits(after, first)  # the order is observable on these inputs


def test_softcap_properties(oracle):
    cap = 30.0
    v = np.concatenate([np.linspace(-200, 200, 40001), [0.0, 1e-30, 1e-3, 29.99, 1e9, -1e9]]).astype(np.float32)
    c = oracle.softcap(v, cap)
    assert np.all(np.abs(c) <= cap)
    assert same_bits(oracle.softcap(-v, cap), -c)                 # odd
    order = np.argsort(v, kind="stable")
    assert np.all(np.diff(c[order].astype(np.float64)) >= 0)       # monotone
    small = np.abs(v) < 1e-2
    assert np.allclose(c[small], v[small], rtol=1e-6, atol=0)      # slope 1 at 0
    ref = (cap * np.tanh(v.astype(np.float64) / cap)).astype(np.float32)
    ulp = np.spacing(np.abs(ref).astype(np.float32))
    assert np.all(np.abs(c.astype(np.float64) - ref) <= 2 * ulp)
    assert same_bits(oracle.softcap(np.array([np.inf, -np.inf], np.float32), cap), np.array([cap, -cap], np.float32))
    assert np.isnan(oracle.softcap(np.array([np.nan], np.float32), cap)[0])


def test_ffn_block_is_the_composition(oracle):
    dim, hidden, eps = 256, 512, 1e-6
    g = synth.q4_0(5, "g", hidden * dim)
    u = synth.q4_0(5, "u", hidden * dim)
    d = synth.q4_0(5, "d", dim * hidden)
    npre, npost = synth.norm_weight(5, "a", dim), synth.norm_weight(5, "b", dim)
    x = synth.activations(5, "x", dim, 4.0)
    got = oracle.ffn_block(Q4_0, g, Q4_0, u, Q4_0, d, npre, npost, x, dim, hidden, eps)
    xb = oracle.rmsnorm(x, npre, eps)
    h = np.array([oracle.gelu(float(v)) for v in oracle.matmul(Q4_0, g, xb, hidden, dim)], np.float32)
    h = h * oracle.matmul(Q4_0, u, xb, hidden, dim)
    y = oracle.rmsnorm(oracle.matmul(Q4_0, d, h, dim, hidden), npost, eps)
    assert same_bits(got, x + y)
    x64, b64 = oracle.ffn_block_exact(Q4_0, g, Q4_0, u, Q4_0, d, npre, npost, x, dim, hidden, eps)
    assert np.all(np.abs(got - x64) <= 1e-5 * b64)
    # swapping the two norm weights is caught by the bound
    bad = oracle.ffn_block(Q4_0, g, Q4_0, u, Q4_0, d, npost, npre, x, dim, hidden, eps)
    assert not np.all(np.abs(bad - x64) <= 1e-5 * b64)


@pytest.mark.parametrize("cap", [0.0, 30.0])
def test_lm_head_is_the_composition(oracle, cap):
    vocab, dim, eps = 4096, 256, 1e-6
    w = synth.q8_0(6, "w", vocab * dim, dscale=0.002)
    norm = synth.norm_weight(6, "n", dim)
    x = synth.activations(6, "x", dim)
    logits, idx = oracle.lm_head(Q8_0, w, norm, x, vocab, dim, eps, cap)
    ref = oracle.matmul(Q8_0, w, oracle.rmsnorm(x, norm, eps), vocab, dim)
    if cap > 0:
        ref = oracle.softcap(ref, cap)
    assert same_bits(logits, ref)
    assert idx == oracle.argmax(ref)
    l64, b64 = oracle.lm_head_exact(Q8_0, w, norm, x, vocab, dim, eps, cap)
    assert np.all(np.abs(logits - l64) <= 1e-5 * b64)
    assert int(np.argmax(l64)) == idx


# ------------------------------------------------------------ attention ---
# Llama.kt:198-218.  Pins: a single position returns V exactly; equal keys give
# the mean of V; GQA reads kv head h / kv_mul; rows before the window start are
# never read; fp64 brute force within the propagated bound.

def _att_inputs(n_heads, n_kv, hs, rows, seed=21):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(n_heads * hs).astype(np.float32)
    kc = rng.standard_normal(rows * n_kv * hs).astype(np.float32)
    vc = rng.standard_normal(rows * n_kv * hs).astype(np.float32)
    return q, kc, vc


def test_attention_single_position_returns_v(oracle):
    q, kc, vc = _att_inputs(4, 2, 64, 1)
    out = oracle.attention(q, kc, vc, 4, 2, 64, 0)
    v = vc.reshape(1, 2, 64)[0]
    assert same_bits(out, np.stack([v[0], v[0], v[1], v[1]]))


def test_attention_equal_keys_average_v(oracle):
    n_heads, n_kv, hs, rows = 2, 1, 32, 100
    q, _, vc = _att_inputs(n_heads, n_kv, hs, rows)
    kc = np.tile(np.random.default_rng(3).standard_normal(hs).astype(np.float32), rows)
    out = oracle.attention(q, kc, vc, n_heads, n_kv, hs, rows - 1)
    mean = vc.reshape(rows, hs).astype(np.float64).mean(axis=0)
    assert np.allclose(out, mean, rtol=0, atol=1e-5)


def test_attention_gqa_mapping_and_window(oracle):
    n_heads, n_kv, hs, rows = 8, 2, 64, 50
    q, kc, vc = _att_inputs(n_heads, n_kv, hs, rows)
    v = vc.reshape(rows, n_kv, hs)
    v[:, 0, :] = 1.0
    v[:, 1, :] = 2.0
    kc.reshape(rows, n_kv, hs)[:20] = np.nan  # before the window: never read
    v[:20] = np.nan
    out = oracle.attention(q, kc, v.reshape(-1), n_heads, n_kv, hs, rows - 1, 20)
    want = np.repeat([1.0, 2.0], n_heads // n_kv)[:, None] * np.ones(hs)
    assert np.allclose(out, want, rtol=1e-6, atol=0)


@pytest.mark.parametrize("n_heads,n_kv,hs,rows,start", [(4, 4, 64, 37, 0), (8, 2, 256, 300, 0),
                                                        (8, 1, 128, 500, 250), (2, 1, 80, 64, 10)])
def test_attention_vs_fp64(oracle, n_heads, n_kv, hs, rows, start):
    q, kc, vc = _att_inputs(n_heads, n_kv, hs, rows)
    out = oracle.attention(q, kc, vc, n_heads, n_kv, hs, rows - 1, start)
    o64, b64 = oracle.attention_exact(q, kc, vc, n_heads, n_kv, hs, rows - 1, start)
    assert np.all(np.abs(out - o64) <= 1e-5 * b64)
    # the bound is not vacuous: reading kv head h % n_kv instead breaks it when heads share kv heads
    if n_heads != n_kv and n_kv > 1:
        bad = np.stack([oracle.attention(q[h * hs:(h + 1) * hs], np.ascontiguousarray(
            kc.reshape(rows, n_kv, hs)[:, h % n_kv]), np.ascontiguousarray(vc.reshape(rows, n_kv, hs)[:, h % n_kv]),
            1, 1, hs, rows - 1, start)[0] for h in range(n_heads)])
        assert not np.all(np.abs(bad - o64) <= 1e-5 * b64)


# ------------------------------------------------------------------- MoE ---
# Llama.kt:269-337 with MutableFloatTensor.kt:54-66.  The oracle's or_moe /
# or_moe_exact are pinned three ways: (1) or_moe_exact against a numpy fp64
# brute force over npref's independently decoded expert slabs (gate rows at
# e*2*ff*dim, up rows after them, down at e*dim*ff), to 1e-12; (2) or_moe bit for
# bit against its own composition from the pinned pieces (oracle.matmul at the
# slab offsets, gelu, the product with up, saxpy in top-k order); (3) mutations
# of the slab layout and of the gate weights, which the comparison must reject.

def _gelu64(v: np.ndarray) -> np.ndarray:
    v = v.astype(np.float64)
    return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))


def _moe_fp64(t, gate_up, down, X, ids, w, dim, ff, gu_stride=None, swap_halves=False):
    """numpy fp64 restatement of Llama.kt:300-337 from npref's decode.  Returns
    (Y, scale) with scale = sum_j |w_j| sum_i |Wd[r, i] h_i| (the size of the
    terms, for a relative tolerance)."""
    GU = npref.dequant(t, gate_up).astype(np.float64)
    DN = npref.dequant(t, down).astype(np.float64)
    stride = 2 * ff * dim if gu_stride is None else gu_stride
    T, k = ids.shape
    Y = np.zeros((T, dim))
    S = np.zeros((T, dim))
    for tok in range(T):
        x = X[tok].astype(np.float64)
        for j in range(k):
            e = int(ids[tok, j])
            slab = GU[e * stride:e * stride + 2 * ff * dim].reshape(2 * ff, dim)
            g, u = slab[:ff] @ x, slab[ff:] @ x
            if swap_halves:
                g, u = u, g
            h = _gelu64(g) * u
            Wd = DN[e * dim * ff:(e + 1) * dim * ff].reshape(dim, ff)
            Y[tok] += float(w[tok, j]) * (Wd @ h)
            S[tok] += abs(float(w[tok, j])) * (np.abs(Wd) @ np.abs(h))
    return Y, S


def _moe_case(E=6, dim=128, ff=64, T=3, k=3, seed=31):
    gate_up = synth.q4_k(seed, "gu", E * 2 * ff * dim)
    down = synth.q4_k(seed, "dn", E * dim * ff)
    X = synth.activations(seed, "x", T * dim).reshape(T, dim)
    logits = synth.activations(seed, "lg", T * E).reshape(T, E)
    return gate_up, down, X, logits


@pytest.mark.parametrize("E,dim,ff,T,k", [(4, 64, 64, 2, 2), (6, 128, 64, 3, 3), (8, 128, 64, 2, 3)])
def test_moe_exact_matches_numpy_fp64(oracle, E, dim, ff, T, k):
    gate_up, down, X, logits = _moe_case(E, dim, ff, T, k)
    ids, w = oracle.route(logits, k, True)
    y64, b64 = oracle.moe_exact(Q4_K, gate_up, Q4_K, down, X, ids, w, dim, ff)
    ynp, scale = _moe_fp64(Q4_K, gate_up, down, X, ids, w, dim, ff)
    assert np.all(np.abs(y64 - ynp) <= 1e-12 * scale + 1e-300)
    # the fp32 restatement sits inside the propagated bound around the fp64 value
    y32 = oracle.moe(Q4_K, gate_up, Q4_K, down, X, ids, w, dim, ff)
    assert np.all(np.abs(y32 - ynp) <= 1e-5 * b64)


def test_moe_routing_matches_numpy(oracle):
    # softmax in double over all experts, top-k with ties to the lowest index,
    # then (for the configuration's renormalised gates) w_j / sum of the k picks
    _, _, _, logits = _moe_case(E=32, T=5)
    k = 4
    for renorm in (False, True):
        ids, w = oracle.route(logits, k, renorm)
        for t in range(logits.shape[0]):
            l64 = logits[t].astype(np.float64)
            p = np.exp(l64 - l64.max())
            p = p / p.sum()
            order = np.argsort(-p, kind="stable")[:k]
            assert np.array_equal(ids[t], order)
            want = p[order] / (p[order].sum() if renorm else 1.0)
            assert np.allclose(w[t], want, rtol=1e-6, atol=0)


def test_moe_is_the_composition(oracle):
    E, dim, ff, T, k = 6, 128, 64, 3, 3
    gate_up, down, X, logits = _moe_case(E, dim, ff, T, k)
    ids, w = oracle.route(logits, k, True)
    got = oracle.moe(Q4_K, gate_up, Q4_K, down, X, ids, w, dim, ff)
    for tok in range(T):
        out = np.zeros(dim, np.float32)
        for j in range(k):
            e = int(ids[tok, j])
            gu = oracle.matmul(Q4_K, gate_up, X[tok], 2 * ff, dim, this_offset=e * 2 * ff * dim)
            g, u = gu[:ff], gu[ff:]
            h = np.array([oracle.gelu(float(v)) for v in g], np.float32) * u
            dn = oracle.matmul(Q4_K, down, h, dim, ff, this_offset=e * dim * ff)
            # saxpyInPlace: out[i] = a * that[i] + out[i], each step rounded to fp32
            out = (np.float32(w[tok, j]) * dn + out).astype(np.float32)
        assert same_bits(got[tok], out)


@pytest.mark.parametrize("mutation", ["swap_gate_up", "gu_stride_ff_dim", "not_renormalised", "gates_misassigned"])
def test_mutation_moe_layout_detected(oracle, mutation):
    E, dim, ff, T, k = 6, 128, 64, 3, 3
    gate_up, down, X, logits = _moe_case(E, dim, ff, T, k)
    ids, w = oracle.route(logits, k, True)
    y64, b64 = oracle.moe_exact(Q4_K, gate_up, Q4_K, down, X, ids, w, dim, ff)
    if mutation == "swap_gate_up":
        bad, _ = _moe_fp64(Q4_K, gate_up, down, X, ids, w, dim, ff, swap_halves=True)
    elif mutation == "gu_stride_ff_dim":
        bad, _ = _moe_fp64(Q4_K, gate_up, down, X, ids, w, dim, ff, gu_stride=ff * dim)
    elif mutation == "not_renormalised":
        _, w_raw = oracle.route(logits, k, False)
        bad, _ = _moe_fp64(Q4_K, gate_up, down, X, ids, w_raw, dim, ff)
    else:  # gate weight j applied to another slot's expert
        bad, _ = _moe_fp64(Q4_K, gate_up, down, X, ids[:, ::-1].copy(), w, dim, ff)
    assert not np.all(np.abs(bad - y64) <= 1e-5 * b64)
