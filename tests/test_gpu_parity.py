"""GPU parity of libg4hip.so against the CPU oracle.

Bars (written into each check):
  * dequantised weights (get): bit-exact fp32;
  * every dot product: |y - exact| <= 1e-5 * sum|w_i x_i| (+1e-30), exact = fp64 sum
    over the exactly dequantised weights (the reference's restated vectorDot meets
    the same bound, tests/test_oracle_pins.py);
  * argmax indices, routing ids and routing weights: exact.
"""
import numpy as np
import pytest

import synth
from conftest import announce

pytestmark = pytest.mark.gpu

Q8_0, Q4_0, Q4_K, Q5_K, Q6_K, F16, BF16, F32 = 8, 2, 12, 13, 14, 1, 30, 0
ALL = [Q8_0, Q4_0, Q4_K, Q5_K, Q6_K, F16, BF16, F32]
TOL = 1e-5


def same_bits(a, b) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn]))


def assert_dots(y, exact, absum, what=""):
    y = np.asarray(y, np.float64)
    err = np.abs(y - exact)
    bound = TOL * absum + 1e-30
    bad = np.nonzero(err > bound)[0]
    assert bad.size == 0, "%s: %d rows out of tolerance, first %d: y=%r exact=%r bound=%r" % (
        what, bad.size, bad[0], y[bad[0]], exact[bad[0]], bound[bad[0]])


def upload(g4, ctx, t, raw, n):
    return g4.FloatTensorFactory.create(ctx, t, raw, n)


# ----------------------------------------------------------------- dequant ---

@pytest.mark.parametrize("t", ALL)
def test_dequant_bit_exact(g4, ctx, oracle, t):
    announce("dequant type=%d" % t)
    n = 256 * 96
    raw = synth.weights(41, "dq%d" % t, t, n)
    w = upload(g4, ctx, t, raw, n)
    assert same_bits(w.dequant(0, n), oracle.dequant(t, raw, 0, n))
    assert same_bits(w.dequant(77, 1000), oracle.dequant(t, raw, 77, 1000))
    assert same_bits([w.get(5), w.get(n - 1)], [oracle.get(t, raw, 5), oracle.get(t, raw, n - 1)])


def test_dequant_every_fp16_scale(g4, ctx, oracle):
    """All 65536 fp16 patterns as Q8_0 scales with q = 1 and q = -3: w = q * d."""
    announce("dequant fp16 scales")
    nb = 65536
    blk = np.zeros((nb, 34), np.uint8)
    blk[:, 0:2] = np.arange(nb, dtype=np.uint32).astype(np.uint16).view(np.uint8).reshape(nb, 2)
    blk[:, 2] = 1
    blk[:, 3] = np.uint8(0xFD)  # -3
    raw = blk.reshape(-1)
    w = upload(g4, ctx, Q8_0, raw, nb * 32)
    got = w.dequant(0, nb * 32).reshape(nb, 32)
    want = oracle.dequant(Q8_0, raw, 0, nb * 32).reshape(nb, 32)
    assert same_bits(got[:, :2], want[:, :2])
    d = np.arange(nb, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    assert same_bits(got[:, 0], d)


def test_dequant_f16_every_pattern(g4, ctx, oracle):
    announce("dequant f16 patterns")
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    w = upload(g4, ctx, F16, raw, 65536)
    assert same_bits(w.dequant(0, 65536), oracle.fp16_to_f32_array(raw))


# ------------------------------------------------------------------ matmul ---

SHAPES = [
    # (dim0, dim1, this_offset_rows, description)
    (64, 2048, 0, "aligned 2048"),
    (37, 1024, 3, "aligned 1024, odd rows, row offset"),
    (19, 8192, 1, "multi-pass 8192"),
    (24, 1408, 1, "1408 (Q4_K rows straddle super-blocks)"),
    (13, 1536, 2, "1536 (24 chunks, x read at use)"),
    (9, 640, 0, "short rows (16-lane groups)"),
]


@pytest.mark.parametrize("t", ALL)
@pytest.mark.parametrize("shape", SHAPES, ids=[s[3] for s in SHAPES])
def test_matmul_fast_path(g4, ctx, oracle, t, shape):
    dim0, dim1, roff, _ = shape
    announce("matmul type=%d shape=%r" % (t, shape))
    n = (dim0 + roff + 1) * dim1
    n = (n + 255) // 256 * 256
    raw = synth.weights(42, "mm%d.%d" % (t, dim1), t, n)
    x = synth.activations(42, "x%d" % dim1, dim1)
    w = upload(g4, ctx, t, raw, n)
    off = roff * dim1
    y = np.empty(dim0, np.float32)
    w.matmul(x, y, dim0, dim1, off)
    ex, ab = oracle.matmul_exact(t, raw, x, dim0, dim1, off)
    assert_dots(y, ex, ab, "type %d %r" % (t, shape))
    ref = oracle.matmul(t, raw, x, dim0, dim1, off)
    assert_dots(ref, ex, ab, "oracle")


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q5_K])
def test_matmul_x_at_use_many_tiles(g4, ctx, oracle, t):
    """17 chunks per row (8 lanes x 3 chunks, x read from LDS per chunk), with
    enough rows that every wave runs three tiles and the last one is partial."""
    dim0, dim1 = 36001, 1088
    announce("matmul x-at-use type=%d %dx%d" % (t, dim0, dim1))
    n = (dim0 * dim1 + 255) // 256 * 256
    raw = synth.weights(44, "xl%d" % t, t, n)
    x = synth.activations(44, "xl", dim1)
    w = upload(g4, ctx, t, raw, n)
    y = np.empty(dim0, np.float32)
    w.matmul(x, y, dim0, dim1, 0)
    ex, ab = oracle.matmul_exact(t, raw, x, dim0, dim1, 0)
    assert_dots(y, ex, ab, "x at use type %d" % t)


GENERIC = [(5, 1000, 7), (3, 33, 1), (4, 2048, 32), (2, 96, 64 + 32), (6, 17, 0), (1, 5, 250)]


@pytest.mark.parametrize("t", ALL)
@pytest.mark.parametrize("g", GENERIC, ids=[str(g) for g in GENERIC])
def test_matmul_unaligned_offsets(g4, ctx, oracle, t, g):
    """Offsets / lengths off the 64-element grid (the reference's scalar head/tail)."""
    dim0, dim1, off = g
    announce("matmul generic type=%d %r" % (t, g))
    n = ((off + dim0 * dim1 + 511) // 256) * 256
    raw = synth.weights(43, "gen%d" % t, t, n)
    x = synth.activations(43, "xg", dim1)
    w = upload(g4, ctx, t, raw, n)
    y = np.empty(dim0, np.float32)
    w.matmul(x, y, dim0, dim1, off)
    ex, ab = oracle.matmul_exact(t, raw, x, dim0, dim1, off)
    assert_dots(y, ex, ab, "generic %d %r" % (t, g))


def test_matmul_f16_vector_decode_semantics(g4, ctx, oracle):
    """Subnormal / non-finite fp16 weights: the dot follows the vector path's
    decode for j < dim1 & ~15 and the exact decode in the tail (F16FloatTensor.kt:43-77)."""
    announce("f16 special weights")
    dim1 = 64 + 20
    wts = np.full(2 * dim1, 0x3C00, np.uint16)  # 1.0
    wts[5] = 0x0001                             # subnormal inside the vector part -> 0
    wts[dim1 - 2] = 0x0003                      # subnormal in the tail -> exact
    wts[dim1 + 7] = 0x7C00                      # +inf in the vector part -> 65536
    x = np.ones(dim1, np.float32)
    w = upload(g4, ctx, F16, wts, 2 * dim1)
    y = np.empty(2, np.float32)
    w.matmul(x, y, 2, dim1)
    exp0 = (dim1 - 2) + 3 * 2.0 ** -24  # 82 ones, one flushed subnormal, one exact tail subnormal
    exp1 = (dim1 - 1) + 65536.0
    assert abs(y[0] - exp0) <= TOL * dim1 and abs(y[1] - exp1) <= TOL * (dim1 + 65536)
    ref = oracle.matmul(F16, wts, x, 2, dim1)
    assert abs(ref[0] - exp0) <= TOL * dim1 and abs(ref[1] - exp1) <= TOL * (dim1 + 65536)


def test_matmul_dev_matches_host(g4, ctx, oracle):
    import torch
    announce("matmul_dev")
    dim0, dim1 = 128, 2048
    raw = synth.weights(44, "dev", Q4_0, dim0 * dim1)
    x = synth.activations(44, "x", dim1)
    w = upload(g4, ctx, Q4_0, raw, dim0 * dim1)
    y = np.empty(dim0, np.float32)
    w.matmul(x, y, dim0, dim1)
    xd = torch.from_numpy(x).cuda()
    yd = torch.empty(dim0, dtype=torch.float32, device="cuda")
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    try:
        w.matmul_dev(xd, yd, dim0, dim1)
        torch.cuda.synchronize()
    finally:
        ctx.set_stream(None)
    assert same_bits(yd.cpu().numpy(), y)


def test_concurrent_contexts_share_weights(g4, ctx, oracle):
    """Several generate calls may run at once on one model (GemmaModel.kt:73): four
    threads, each with its own context, run matmul (Q4_K and Q8_0) and the routed MoE
    on weights uploaded once, at the same time (ctypes drops the GIL during the
    calls).  Every result equals the one the same call gives alone, bit for bit."""
    import threading
    announce("concurrent contexts")
    dim0, dim1 = 1024, 2048
    raw_k = synth.weights(57, "ck", Q4_K, dim0 * dim1)
    raw_8 = synth.weights(57, "c8", Q8_0, dim0 * dim1)
    wk = upload(g4, ctx, Q4_K, raw_k, dim0 * dim1)
    w8 = upload(g4, ctx, Q8_0, raw_8, dim0 * dim1)
    E, D, FF, K = 16, 512, 256, 4
    gu = synth.q4_k(57, "gu", E * 2 * FF * D)
    dn = synth.q4_k(57, "dn", E * D * FF)
    wgu = upload(g4, ctx, Q4_K, gu, E * 2 * FF * D)
    wdn = upload(g4, ctx, Q4_K, dn, E * D * FF)
    xs = [synth.activations(57, "x%d" % i, dim1) for i in range(6)]
    lgs = [synth.activations(57, "lg%d" % i, 2 * E).reshape(2, E) for i in range(6)]
    Xs = [synth.activations(57, "X%d" % i, 2 * D).reshape(2, D) for i in range(6)]
    alone = []
    for i in range(6):
        yk = np.empty(dim0, np.float32)
        y8 = np.empty(dim0, np.float32)
        wk.matmul(xs[i], yk, dim0, dim1)
        w8.matmul(xs[i], y8, dim0, dim1)
        Y, ids, gw = g4.moe_routed(ctx, wgu, wdn, Xs[i], lgs[i], K, True, D, FF)
        alone.append((yk, y8, Y, ids, gw))
    lib = g4.lib()
    bad = []

    def worker(k):
        c = g4.Context(0)
        try:
            for it in range(12):
                i = (k + it) % 6
                yk = np.empty(dim0, np.float32)
                y8 = np.empty(dim0, np.float32)
                g4.check(lib.g4_matmul(c.handle, wk.handle, 0, xs[i].ctypes.data, yk.ctypes.data, dim0, dim1))
                g4.check(lib.g4_matmul(c.handle, w8.handle, 0, xs[i].ctypes.data, y8.ctypes.data, dim0, dim1))
                Y, ids, gw = g4.moe_routed(c, wgu, wdn, Xs[i], lgs[i], K, True, D, FF)
                ref = alone[i]
                if not (same_bits(yk, ref[0]) and same_bits(y8, ref[1]) and same_bits(Y, ref[2])
                        and np.array_equal(ids, ref[3]) and same_bits(gw, ref[4])):
                    bad.append((k, it))
        except Exception as e:  # reported below, in the test's thread
            bad.append((k, repr(e)))
        finally:
            c.close()

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads)
    assert not bad, bad[:5]


def test_range_errors_on_device(g4, ctx):
    announce("range errors")
    raw = synth.weights(45, "err", Q8_0, 64 * 32)
    w = upload(g4, ctx, Q8_0, raw, 64 * 32)
    x = np.zeros(64, np.float32)
    y = np.zeros(64, np.float32)
    with pytest.raises(g4.IndexOutOfBoundsException):
        w.matmul(x, y, 33, 64)
    with pytest.raises(g4.IndexOutOfBoundsException):
        w.matmul(x, y, 32, 64, 1)
    with pytest.raises(g4.IllegalArgumentException):
        g4.FloatTensorFactory.create(ctx, Q8_0, raw[:100], 64 * 32)
    with pytest.raises(g4.UnsupportedOperationException):
        g4.FloatTensorFactory.create(ctx, 3, raw, 64 * 32)
    # MoE: more (token, slot) pairs than one launch takes, checked before any copy
    gu = synth.weights(45, "egu", Q8_0, 2 * 2 * 32 * 64)
    wgu = upload(g4, ctx, Q8_0, gu, 2 * 2 * 32 * 64)
    wdn = upload(g4, ctx, Q8_0, gu[: gu.size // 2], 2 * 32 * 64)
    with pytest.raises(g4.IllegalArgumentException):
        g4.moe_dev(ctx, wgu, wdn, 0, 32769, 64, 32, 0, 0, 2, 0)


# -------------------------------------------------------------- workloads ---

def test_q8_0_matvec_2048(g4, ctx, oracle):
    announce("workload q8_0 matvec 2048x2048")
    c = synth.q8_0_matvec_2048()
    w = upload(g4, ctx, Q8_0, c["w"], 2048 * 2048)
    y = np.empty(2048, np.float32)
    w.matmul(c["x"], y, 2048, 2048)
    ex, ab = oracle.matmul_exact(Q8_0, c["w"], c["x"], 2048, 2048)
    assert_dots(y, ex, ab, "q8_0 2048")


def _ffn_reference(oracle, c):
    dim, hidden = c["dim"], c["hidden"]
    gu = np.concatenate([c["gate"], c["up"]])
    ids = np.zeros((1, 1), np.int32)
    one = np.ones((1, 1), np.float32)
    y64, bound = oracle.moe_exact(Q4_0, gu, Q4_0, c["down"], c["x"].reshape(1, dim), ids, one, dim, hidden)
    return y64[0], bound[0]


def test_gelu_through_identity_gate_up(g4, ctx, oracle):
    """gelu itself (Llama.kt:23-25, a double tanh by fdlibm's steps): with BF16
    identity gate and up matrices, h_i = gelu(x_i) * x_i exactly, so h is compared
    bit for bit with the oracle's gelu over x spanning its regimes (cancellation of
    1 + tanh near x = -6, saturation, tiny and huge x).  The device's expm1 and the
    C library's may differ in a last bit, which reaches the float result only in
    rare halfway cases."""
    announce("gelu through identity gate/up")
    n = 4096
    rng = np.random.default_rng(63)
    x = np.concatenate([np.linspace(-12, 12, n // 2), 10.0 ** rng.uniform(-30, 1.5, n // 2 - 8) *
                        rng.choice([-1.0, 1.0], n // 2 - 8),
                        [0.0, -0.0, 1e-40, -1e-40, 3e38, -3e38, 40.0, -40.0]]).astype(np.float32)
    eye = np.zeros((n, n), np.uint16)
    eye[np.arange(n), np.arange(n)] = 0x3F80  # bf16 1.0
    w = upload(g4, ctx, BF16, eye.view(np.uint8).reshape(-1), n * n)
    h = g4.ffn_gate_up(ctx, w, w, x, n, n)
    with np.errstate(over="ignore"):  # gelu(3e38) * 3e38 overflows to inf on both sides
        ref = np.array([np.float32(oracle.gelu(float(v))) * v for v in x], np.float32)
    fin = np.isfinite(ref)
    assert np.count_nonzero(h[fin].view(np.uint32) != ref[fin].view(np.uint32)) <= 1
    assert same_bits(h[~fin], ref[~fin])


def test_q4_0_ffn_one_token(g4, ctx, oracle):
    announce("workload q4_0 ffn 8192x2048")
    c = synth.q4_0_ffn()
    dim, hidden = c["dim"], c["hidden"]
    wg = upload(g4, ctx, Q4_0, c["gate"], hidden * dim)
    wu = upload(g4, ctx, Q4_0, c["up"], hidden * dim)
    wd = upload(g4, ctx, Q4_0, c["down"], dim * hidden)
    y = g4.ffn(ctx, wg, wu, wd, c["x"], dim, hidden)
    y64, bound = _ffn_reference(oracle, c)
    assert_dots(y, y64, bound, "ffn")
    # each matvec on its own too
    g = np.empty(hidden, np.float32)
    wg.matmul(c["x"], g, hidden, dim)
    ex, ab = oracle.matmul_exact(Q4_0, c["gate"], c["x"], hidden, dim)
    assert_dots(g, ex, ab, "gate")


def test_q8_0_lm_head_argmax(g4, ctx, oracle):
    announce("workload q8_0 lm head 262144x2048 + argmax")
    c = synth.q8_0_lm_head()
    V, D = c["dim0"], c["dim1"]
    w = upload(g4, ctx, Q8_0, c["w"], V * D)
    logits = np.empty(V, np.float32)
    idx = w.matmul_argmax(c["x"], V, D, logits=logits)
    ex, ab = oracle.matmul_exact(Q8_0, c["w"], c["x"], V, D)
    assert_dots(logits, ex, ab, "lm head")
    # the argmax of the GPU's own logits is the sequential-scan argmax of them
    assert idx == oracle.argmax(logits)
    # and equals the exact argmax: the top-1/top-2 gap exceeds both error bounds
    order = np.argsort(-ex, kind="stable")
    gap = ex[order[0]] - ex[order[1]]
    assert gap > 2 * TOL * max(ab[order[0]], ab[order[1]]), "fixture gap too small to pin the argmax"
    assert idx == int(order[0])
    # index-only call (logits not returned)
    assert w.matmul_argmax(c["x"], V, D) == idx


@pytest.mark.parametrize("D", [1088, 2112, 640])
def test_matmul_argmax_winner_in_every_wave(g4, ctx, oracle, D):
    """A vocabulary-sized arg-max launch (65536 rows: one 8-wave workgroup per CU;
    with 1088 columns each wave takes a contiguous range of 32 rows, wave w of every
    workgroup covering rows 8192 w .. 8192 w + 8191; 2112 and 640 columns take the
    64- and 16-lane row groups).  x is made equal to row 8192 w + 5, so that row
    wins, for each w; then a copy of the winner at a lower row in another wave (same
    position in its tile, so the two dots are bit-equal) must win the tie."""
    V = 65536
    announce("matmul_argmax 8-wave groups %dx%d" % (V, D))
    n = V * D
    raw = synth.weights(61, "am8.%d" % D, Q8_0, n)
    w = upload(g4, ctx, Q8_0, raw, n)
    for wave in range(8):
        r = 8192 * wave + 5
        x = oracle.dequant(Q8_0, raw, r * D, D)
        logits = np.empty(V, np.float32)
        idx = w.matmul_argmax(x, V, D, logits=logits)
        ex, ab = oracle.matmul_exact(Q8_0, raw, x, V, D)
        assert_dots(logits, ex, ab, "argmax wave %d" % wave)
        order = np.argsort(-ex, kind="stable")
        assert int(order[0]) == r, "fixture: row %d is not the exact winner" % r
        assert ex[order[0]] - ex[order[1]] > 2 * TOL * max(ab[order[0]], ab[order[1]])
        assert idx == r, (wave, idx)
    # tie across waves: row 8192 * 2 + 5 becomes a copy of row 8192 * 6 + 5
    bpr = D // 32 * 34
    tied = np.array(raw, dtype=np.uint8, copy=True)
    win, low = 8192 * 6 + 5, 8192 * 2 + 5
    tied[low * bpr:(low + 1) * bpr] = tied[win * bpr:(win + 1) * bpr]
    wt = upload(g4, ctx, Q8_0, tied, n)
    x = oracle.dequant(Q8_0, tied, win * D, D)
    logits = np.empty(V, np.float32)
    idx = wt.matmul_argmax(x, V, D, logits=logits)
    assert logits[low] == logits[win]
    assert idx == low == oracle.argmax(logits)


@pytest.mark.parametrize("m", [1, 8, 32, 64])
def test_q4_k_batched(g4, ctx, oracle, m):
    announce("workload q4_k batched M=%d" % m)
    c = synth.q4_k_batched(m)
    R, D = c["dim0"], c["dim1"]
    w = upload(g4, ctx, Q4_K, c["w"], R * D)
    Y = w.matmul_batch(c["x"], R, D)
    # every row of every token (a tile or row-range indexing error that only the
    # full grid reaches shows here)
    for i in range(m):
        ex, ab = oracle.matmul_exact(Q4_K, c["w"], c["x"][i], R, D)
        assert_dots(Y[i], ex, ab, "batched m=%d token %d" % (m, i))


def _integer_blocks(t, n, seed):
    """Blocks of type t whose weights are all small integers: unit d (and dmin),
    scales and mins in 0..3 (Q6_K: -3..3), every quant field random.  With integer
    x in -3..3 every product and every partial sum of a dot is an exact fp32
    integer (below 2^24 for the sizes used here)."""
    rng = np.random.default_rng(seed)
    one = synth.fp16_bits(np.array([1.0])).view(np.uint8)
    if t == Q8_0:
        raw = synth.q8_0(seed, "int", n).reshape(-1, 34)
        raw[:, 0:2] = one
    elif t == Q4_0:
        raw = synth.q4_0(seed, "int", n).reshape(-1, 18)
        raw[:, 0:2] = one
    elif t in (Q4_K, Q5_K):
        raw = (synth.q4_k if t == Q4_K else synth.q5_k)(seed, "int", n).reshape(n // 256, -1)
        raw[:, 0:2] = one
        raw[:, 2:4] = one
        raw[:, 4:16] = synth.pack_q4k_scales(rng.integers(0, 4, (n // 256, 8)), rng.integers(0, 4, (n // 256, 8)))
    else:
        raw = synth.q6_k(seed, "int", n).reshape(-1, 210)
        raw[:, 192:208] = rng.integers(-3, 4, (n // 256, 16)).astype(np.int8).view(np.uint8)
        raw[:, 208:210] = one
    return raw.reshape(-1)


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("rows,cols", [(64, 2048), (96, 1408), (8, 16384), (40, 512)])
def test_integer_dots_exact(g4, ctx, oracle, t, rows, cols):
    """Integer weights (every quant value at every position, scales and mins
    unpacked) against integer x: every kernel must return the exact dot, so a
    weight unpacked, placed or scaled wrongly shows as an integer error, not as
    rounding.  One column pass (2048), x read at use (1408 = 22 chunks), several
    passes and the wide rows (16384), 16-lane rows (512); Q4_K also through the
    matrix-core kernel (M = 8 and 33)."""
    announce("integer dots type %d %dx%d" % (t, rows, cols))
    n = rows * cols
    raw = _integer_blocks(t, n, 81 + t)
    W = oracle.dequant(t, raw, 0, n).reshape(rows, cols).astype(np.float64)
    assert np.all(W == np.round(W)) and np.max(np.abs(W)) < 512
    rng = np.random.default_rng(82 + cols)
    X = rng.integers(-3, 4, (33, cols)).astype(np.float32)
    w = upload(g4, ctx, t, raw, n)
    y = np.empty(rows, np.float32)
    w.matmul(X[0], y, rows, cols)
    ex = W @ X[0].astype(np.float64)
    assert np.array_equal(y.astype(np.float64), ex), "matvec: %r vs %r" % (y[y != ex][:4], ex[y != ex][:4])
    for m in ((8, 33) if t == Q4_K else (3,)):
        Y = w.matmul_batch(X[:m], rows, cols)
        EX = X[:m].astype(np.float64) @ W.T
        bad = np.argwhere(Y.astype(np.float64) != EX)
        assert bad.size == 0, "batched M=%d: %d wrong, first %r: %r vs %r" % (
            m, len(bad), tuple(bad[0]), Y[tuple(bad[0])], EX[tuple(bad[0])])
    w.free()


def test_integer_dots_exact_sixteen_q_operands(g4, ctx, oracle):
    """The matrix-core kernel with five row tiles per workgroup (200 tokens over
    1280 rows), whose weight operands are 16 q less sum(128 x): integer weights
    and activations give the exact dots there too."""
    announce("integer dots batched 16q operands")
    rows, cols, m = 1280, 2048, 200
    n = rows * cols
    raw = _integer_blocks(Q4_K, n, 93)
    W = oracle.dequant(Q4_K, raw, 0, n).reshape(rows, cols).astype(np.float64)
    assert np.all(W == np.round(W))
    X = np.random.default_rng(94).integers(-3, 4, (m, cols)).astype(np.float32)
    w = upload(g4, ctx, Q4_K, raw, n)
    Y = w.matmul_batch(X, rows, cols)
    EX = X.astype(np.float64) @ W.T
    bad = np.argwhere(Y.astype(np.float64) != EX)
    assert bad.size == 0, "%d wrong, first %r: %r vs %r" % (len(bad), tuple(bad[0]), Y[tuple(bad[0])],
                                                           EX[tuple(bad[0])])
    w.free()


# matrix-core multi-token kernel (M >= 3): partial row and token tiles, several
# column splits (summed by the reduce launch: 4224 and 4096 columns), rows that
# start mid super-block (1408 = 5.5 super-blocks), a row offset, a single
# 64-column group and several token groups (M = 17, 48, 70); M = 2 takes the
# row engine, one segment per token.  Whole slices and row tiles (the unchecked
# form) with column splits: at most 8 tokens (6 x 64 x 4096), three token tiles
# and three splits behind a row offset (40 x 64 x 6144), and the 16 q operands
# (32 tokens over 4096 rows: four row tiles per workgroup, two splits)
@pytest.mark.parametrize("m,rows,dim1,off_rows", [
    (2, 40, 2048, 0), (4, 40, 2048, 0), (17, 34, 4224, 0), (5, 34, 1408, 0), (16, 48, 2048, 3),
    (3, 20, 64, 0), (48, 40, 2048, 0), (70, 24, 4096, 1), (6, 64, 4096, 0), (40, 64, 6144, 2),
    (32, 4096, 4096, 0)])
def test_q4_k_batched_matrix_core_shapes(g4, ctx, oracle, m, rows, dim1, off_rows):
    announce("q4_k batched M=%d rows=%d dim1=%d off_rows=%d" % (m, rows, dim1, off_rows))
    n = (rows + off_rows) * dim1
    raw = synth.weights(52, "mc%d.%d" % (rows, dim1), Q4_K, n)
    X = synth.activations(52, "mcx%d.%d" % (m, dim1), m * dim1).reshape(m, dim1)
    w = upload(g4, ctx, Q4_K, raw, n)
    off = off_rows * dim1
    Y = w.matmul_batch(X, rows, dim1, off)
    for i in range(m):
        ex, ab = oracle.matmul_exact(Q4_K, raw, X[i], rows, dim1, off)
        assert_dots(Y[i], ex, ab, "token %d" % i)


@pytest.mark.parametrize("rows,dim1,m", [(40, 2048, 5), (34, 1408, 5), (1280, 2048, 200)])
def test_q4_k_batched_matrix_core_non_finite_x(g4, ctx, oracle, rows, dim1, m):
    """+inf, NaN and -inf activations in three tokens: those tokens' outputs are
    all non-finite, as the reference's are (inf * w and NaN * w reach every row), and
    the finite tokens, which share the kernel's waves with them, stay within the bound.
    Rows of whole super-blocks (2048), rows that start mid super-block (1408), and
    five row tiles per workgroup (the 16 q operands less sum(128 x))."""
    announce("q4_k batched non-finite x rows=%d dim1=%d m=%d" % (rows, dim1, m))
    raw = synth.weights(54, "mcnf%d" % dim1, Q4_K, rows * dim1)
    X = synth.activations(54, "mcnfx%d" % dim1, m * dim1).reshape(m, dim1)
    X[1, 5] = np.inf
    X[2, dim1 // 3] = np.nan
    X[3, dim1 - 7] = -np.inf
    w = upload(g4, ctx, Q4_K, raw, rows * dim1)
    Y = w.matmul_batch(X, rows, dim1)
    for i in range(m):
        ex, ab = oracle.matmul_exact(Q4_K, raw, X[i], rows, dim1)
        if i in (1, 2, 3):
            assert not np.any(np.isfinite(ex))
            assert not np.any(np.isfinite(Y[i])), "token %d: finite outputs %r" % (i, Y[i][np.isfinite(Y[i])][:4])
        else:
            assert_dots(Y[i], ex, ab, "token %d" % i)


def test_q4_k_batched_matrix_core_wide_range_x(g4, ctx, oracle):
    """x spanning 1e-20..1e20: the three bf16 parts of x are exact at every magnitude."""
    announce("q4_k batched wide-range x")
    m, rows, dim1 = 4, 32, 2048
    raw = synth.weights(53, "mcw", Q4_K, rows * dim1)
    rng = np.random.default_rng(53)
    X = (rng.standard_normal((m, dim1)) * 10.0 ** rng.uniform(-20, 20, (m, dim1))).astype(np.float32)
    w = upload(g4, ctx, Q4_K, raw, rows * dim1)
    Y = w.matmul_batch(X, rows, dim1)
    for i in range(m):
        ex, ab = oracle.matmul_exact(Q4_K, raw, X[i], rows, dim1)
        assert_dots(Y[i], ex, ab, "token %d" % i)


@pytest.mark.parametrize("tokens", [1, 16])
@pytest.mark.parametrize("renorm", [True, False])
def test_moe_route_exact(g4, ctx, oracle, tokens, renorm):
    announce("moe route T=%d renorm=%s" % (tokens, renorm))
    lg = synth.activations(46, "route%d" % tokens, tokens * 128).reshape(tokens, 128)
    scale = None if renorm else np.linspace(0.5, 1.5, 128).astype(np.float32)
    ids, w = g4.moe_route(ctx, lg, 8, renorm, scale)
    rids, rw = oracle.route(lg, 8, renorm, scale)
    assert np.array_equal(ids, rids)
    assert same_bits(w, rw)


_MOE_SLABS = {}


def moe_slabs(g4, ctx, c):
    """The 623 MB of expert slabs of the MoE workload, generated and uploaded once
    for every token count (they do not depend on it)."""
    if "w" not in _MOE_SLABS:
        E, D, FF = c["n_experts"], c["dim"], c["ff"]
        _MOE_SLABS["w"] = (upload(g4, ctx, Q4_K, c["gate_up"], E * 2 * FF * D),
                           upload(g4, ctx, Q4_K, c["down"], E * D * FF))
    return _MOE_SLABS["w"]


# the configured workload (128 experts, top-8, dim 2048, ff 1408): 1, 16 and 24
# tokens take the per-pair launches (24: ten down row blocks of 26 row steps per
# token, the last one partial), 48 and 128 the expert-grouped ones
@pytest.mark.parametrize("tokens", [1, 16, 24, 48, 128])
def test_moe_q4_k(g4, ctx, oracle, tokens):
    announce("workload moe q4_k T=%d" % tokens)
    c = synth.moe_q4_k(tokens)
    E, D, FF, K = c["n_experts"], c["dim"], c["ff"], c["k"]
    wgu, wdn = moe_slabs(g4, ctx, c)
    ids, gw = g4.moe_route(ctx, c["logits"], K, True)
    rids, rw = oracle.route(c["logits"], K, True)
    assert np.array_equal(ids, rids) and same_bits(gw, rw)
    Y = g4.moe(ctx, wgu, wdn, c["x"], ids, gw, D, FF)
    y64, bound = oracle.moe_exact(Q4_K, c["gate_up"], Q4_K, c["down"], c["x"], rids, rw, D, FF)
    assert_dots(Y.reshape(-1), y64.reshape(-1), bound.reshape(-1), "moe T=%d" % tokens)
    # the routing inside the gate+up launch gives the same routing and output bits
    Yr, idr, wr = g4.moe_routed(ctx, wgu, wdn, c["x"], c["logits"], K, True, D, FF)
    assert np.array_equal(idr, rids) and same_bits(wr, rw)
    assert same_bits(Yr, Y)


@pytest.mark.parametrize("case", ["t1", "t5", "t16", "ref_gates", "nan", "ties", "near_ties", "e256", "e300",
                                  "generic", "k_all", "k1", "k3", "k12", "ff2560", "rows100"])
def test_moe_routed(g4, ctx, oracle, case):
    """g4_moe_routed: the routing runs inside the gate+up launch (up to 256 experts,
    rows on the 64-element fast path) or in a launch of its own (more experts, or
    the per-element path); either way the routing equals g4_moe_route's and the
    oracle's exactly, and the output g4_moe's bit for bit.  The down projection
    and weighted sum share one launch for k <= 8 and ff <= 2048 (k1, k3: idle
    waves; rows100: a partial row tile) and take two launches beyond (k12, ff2560).
    near_ties: distinct logits whose probabilities round to one value, so the
    probabilities rank by index where the logits rank the other way."""
    announce("moe routed %s" % case)
    E, D, FF, K, T, renorm, fmt = 16, 512, 256, 4, 3, True, Q4_K
    scale = None
    if case in ("t1", "t5", "t16"):
        T = int(case[1:])
    elif case == "ref_gates":
        renorm = False
        scale = np.linspace(0.25, 2.0, E).astype(np.float32)
    elif case == "e256":
        E, D, FF, K = 256, 128, 64, 8
    elif case == "e300":
        E, D, FF, K = 300, 128, 64, 8
    elif case == "generic":
        D, FF = 96, 64      # gate+up rows of 96 elements: the per-element kernel
    elif case == "k_all":
        E, K = 8, 8
    elif case in ("k1", "k3", "k12"):
        K = int(case[1:])
    elif case == "ff2560":
        E, D, FF = 4, 128, 2560
    elif case == "rows100":
        D, FF = 100, 64
    gu = synth.weights(54, "gu" + case, fmt, E * 2 * FF * D)
    dn = synth.weights(54, "dn" + case, fmt, E * D * FF)
    lg = synth.activations(54, "lg" + case, T * E).reshape(T, E)
    X = synth.activations(54, "X" + case, T * D).reshape(T, D)
    if case == "nan":
        lg[1, 3] = np.nan
    elif case == "ties":
        lg[:, :] = np.round(lg * 2) / 2
        lg[0, :] = 1.0
    elif case == "near_ties":
        lg[:, :] = (np.arange(E) * 1e-9).astype(np.float32)   # exp rounds every difference away
        lg[1, ::3] = 0.5                                      # and a token with clear winners too
    wgu = upload(g4, ctx, fmt, gu, E * 2 * FF * D)
    wdn = upload(g4, ctx, fmt, dn, E * D * FF)
    Yr, idr, wr = g4.moe_routed(ctx, wgu, wdn, X, lg, K, renorm, D, FF, scale)
    rids, rw = oracle.route(lg, K, renorm, scale)
    assert np.array_equal(idr, rids) and same_bits(wr, rw)
    ids, gw = g4.moe_route(ctx, lg, K, renorm, scale)
    Y = g4.moe(ctx, wgu, wdn, X, ids, gw, D, FF)
    assert same_bits(Yr, Y)
    y64, bound = oracle.moe_exact(fmt, gu, fmt, dn, X, rids, rw, D, FF)
    assert_dots(Yr.reshape(-1), y64.reshape(-1), bound.reshape(-1), "moe routed %s" % case)


@pytest.mark.parametrize("fmt", [Q4_K, Q8_0])
def test_moe_batch_equals_tokens_alone(g4, ctx, oracle, fmt):
    """A batch of tokens gives every token the bits it gets alone: alone a token's
    down projection and weighted sum share one launch, in a batch of 16 they take
    the per-pair down launch and the combine; ids chosen by three or more pairs of
    the batch included."""
    announce("moe batch vs alone fmt=%d" % fmt)
    E, D, FF, K, T = 16, 512, 256, 4, 16
    gu = synth.weights(58, "gu", fmt, E * 2 * FF * D)
    dn = synth.weights(58, "dn", fmt, E * D * FF)
    lg = synth.activations(58, "lg", T * E).reshape(T, E)
    X = synth.activations(58, "X", T * D).reshape(T, D)
    wgu = upload(g4, ctx, fmt, gu, E * 2 * FF * D)
    wdn = upload(g4, ctx, fmt, dn, E * D * FF)
    Yb, idb, wb = g4.moe_routed(ctx, wgu, wdn, X, lg, K, True, D, FF)
    assert max(np.bincount(idb.reshape(-1))) >= 3
    for t in range(T):
        Y1, id1, w1 = g4.moe_routed(ctx, wgu, wdn, X[t:t + 1], lg[t:t + 1], K, True, D, FF)
        assert np.array_equal(id1[0], idb[t]) and same_bits(w1[0], wb[t]), t
        assert same_bits(Y1[0], Yb[t]), t
    y64, bound = oracle.moe_exact(fmt, gu, fmt, dn, X, idb, wb, D, FF)
    assert_dots(Yb.reshape(-1), y64.reshape(-1), bound.reshape(-1), "moe batch")


@pytest.mark.parametrize("fmt,T,K,D", [(Q4_K, 16, 8, 512), (Q4_K, 5, 3, 512), (Q4_K, 32, 8, 512),
                                       (Q4_K, 7, 1, 100), (Q4_0, 24, 8, 256), (Q8_0, 33, 6, 192),
                                       (Q5_K, 9, 8, 128)])
def test_moe_fused_down_tokens(g4, ctx, oracle, fmt, T, K, D):
    """Down rows of 17..24 chunks (ff = 1408 here) for 2..32 Q4_K tokens (more run
    the experts grouped) and any count of the other formats: one launch
    does the down projection and the weighted sum, workgroup (row block, token)
    with one wave per slot and several 8-row steps per wave (partial last blocks,
    idle slot waves for k < 8, rows that end inside a step at D = 100).  Within
    the bound of the oracle, every token's output bit-equal to the token run
    alone (whose down projection is the one-token fused launch), and out-of-range
    ids add zero rows."""
    import torch
    announce("moe fused down fmt=%d T=%d K=%d D=%d" % (fmt, T, K, D))
    E, FF = 12, 1408
    gu = synth.weights(61, "gu%d" % D, fmt, E * 2 * FF * D)
    dn = synth.weights(61, "dn%d" % D, fmt, E * D * FF)
    lg = synth.activations(61, "lg%d.%d" % (T, K), T * E).reshape(T, E)
    X = synth.activations(61, "X%d.%d" % (T, D), T * D).reshape(T, D)
    wgu = upload(g4, ctx, fmt, gu, E * 2 * FF * D)
    wdn = upload(g4, ctx, fmt, dn, E * D * FF)
    Yb, idb, wb = g4.moe_routed(ctx, wgu, wdn, X, lg, K, True, D, FF)
    y64, bound = oracle.moe_exact(fmt, gu, fmt, dn, X, idb, wb, D, FF)
    assert_dots(Yb.reshape(-1), y64.reshape(-1), bound.reshape(-1), "moe fused down")
    for t in sorted({0, T // 2, T - 1}):
        Y1, id1, w1 = g4.moe_routed(ctx, wgu, wdn, X[t:t + 1], lg[t:t + 1], K, True, D, FF)
        assert np.array_equal(id1[0], idb[t]) and same_bits(w1[0], wb[t]), t
        assert same_bits(Y1[0], Yb[t]), t
    bad = idb.copy()
    bad[0, K - 1] = -1
    bad[T - 1, 0] = E
    d_Y = torch.full((T, D), float("nan"), dtype=torch.float32, device="cuda")
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    try:
        g4.moe_dev(ctx, wgu, wdn, torch.from_numpy(X).cuda(), T, D, FF, torch.from_numpy(bad).cuda(),
                   torch.from_numpy(wb).cuda(), K, d_Y)
        torch.cuda.synchronize()
    finally:
        ctx.set_stream(None)
    ids0, w0 = bad.copy(), wb.copy()
    off = (bad < 0) | (bad >= E)
    ids0[off] = 0
    w0[off] = 0.0
    y64, bound = oracle.moe_exact(fmt, gu, fmt, dn, X, ids0, w0, D, FF)
    assert_dots(d_Y.cpu().numpy().reshape(-1), y64.reshape(-1), bound.reshape(-1), "moe fused down, bad ids")


@pytest.mark.parametrize("fmt,T,K,D,E,case", [(Q4_K, 16, 8, 2048, 32, ""), (Q4_K, 2, 1, 1088, 16, ""),
                                              (Q4_K, 32, 3, 2048, 16, ""), (Q8_0, 5, 8, 1088, 8, ""),
                                              (Q4_0, 16, 8, 2048, 256, ""), (Q5_K, 7, 6, 1536, 16, ""),
                                              (Q6_K, 3, 8, 2048, 16, ""), (Q4_K, 6, 4, 2048, 16, "nan")])
def test_moe_gate_up_slot_waves(g4, ctx, oracle, fmt, T, K, D, E, case):
    """Gate+up of 2 or more tokens (up to 32 of Q4_K, where more run the experts
    grouped) with rows of 17..32 chunks: workgroup (row
    block, token), one wave per slot, routing once per workgroup in 512 threads
    (up to 256 experts; "nan": a NaN logit, the reference's scans).  The routing
    equals the oracle's exactly, the output is within the oracle's bound, equal
    bit for bit to routing first and then g4_moe (the ids path of the same
    launch) and, per token, to the token run alone (the per-pair launch)."""
    announce("moe gate+up slot waves fmt=%d T=%d K=%d D=%d E=%d %s" % (fmt, T, K, D, E, case))
    FF = 256
    gu = synth.weights(62, "gu%d.%d" % (D, E), fmt, E * 2 * FF * D)
    dn = synth.weights(62, "dn%d.%d" % (D, E), fmt, E * D * FF)
    lg = synth.activations(62, "lg%d.%d.%d" % (T, K, E), T * E).reshape(T, E)
    X = synth.activations(62, "X%d.%d" % (T, D), T * D).reshape(T, D)
    if case == "nan":
        lg[1, 5] = np.nan
    wgu = upload(g4, ctx, fmt, gu, E * 2 * FF * D)
    wdn = upload(g4, ctx, fmt, dn, E * D * FF)
    Yr, idr, wr = g4.moe_routed(ctx, wgu, wdn, X, lg, K, True, D, FF)
    rids, rw = oracle.route(lg, K, True)
    assert np.array_equal(idr, rids) and same_bits(wr, rw)
    Y = g4.moe(ctx, wgu, wdn, X, rids, rw, D, FF)
    assert same_bits(Yr, Y)
    y64, bound = oracle.moe_exact(fmt, gu, fmt, dn, X, rids, rw, D, FF)
    assert_dots(Yr.reshape(-1), y64.reshape(-1), bound.reshape(-1), "moe gate+up slot waves")
    for t in sorted({0, T - 1}):
        Y1, id1, w1 = g4.moe_routed(ctx, wgu, wdn, X[t:t + 1], lg[t:t + 1], K, True, D, FF)
        assert np.array_equal(id1[0], idr[t]) and same_bits(w1[0], wr[t]), t
        assert same_bits(Y1[0], Yr[t]), t


@pytest.mark.parametrize("case", ["t64", "t80_e8", "ff384", "nonfinite", "ref_gates"])
def test_moe_grouped_by_expert(g4, ctx, oracle, case):
    """Calls of 41 or more Q4_K tokens run each expert once for all of its (token,
    slot) pairs on the matrix cores (3 x bf16 products, fp32 sums).  The routed
    and the id-taking entry points give the same bits; every output is within the
    bound; a token alone (row kernels) rounds differently but shares the bound.
    t80_e8: ten pairs per expert on average, so experts take two or more passes
    of sixteen pairs; ff384: down rows of 384 columns, every second one starting half
    way into a super-block (staged at its group pair); nonfinite: +inf, NaN and -inf activations reach only
    their own tokens; ref_gates: un-renormalised gates times a per-expert down
    scale (Llama.kt:300-337)."""
    announce("moe grouped %s" % case)
    E, D, FF, K, T = 32, 512, 256, 4, 64
    renorm, scale = True, None
    if case == "ref_gates":
        renorm, scale = False, np.linspace(0.25, 2.0, E).astype(np.float32)
    if case == "t80_e8":
        E, K, T = 8, 1, 80
    elif case == "ff384":
        FF = 384
    gu = synth.q4_k(61, "gu" + case, E * 2 * FF * D)
    dn = synth.q4_k(61, "dn" + case, E * D * FF)
    lg = synth.activations(61, "lg" + case, T * E).reshape(T, E)
    X = synth.activations(61, "X" + case, T * D).reshape(T, D)
    bad = {}
    if case == "nonfinite":
        X[3, 7] = np.inf
        X[10, 300] = np.nan
        X[40, D - 1] = -np.inf
        bad = {3, 10, 40}
    wgu = upload(g4, ctx, Q4_K, gu, E * 2 * FF * D)
    wdn = upload(g4, ctx, Q4_K, dn, E * D * FF)
    Yr, idr, wr = g4.moe_routed(ctx, wgu, wdn, X, lg, K, renorm, D, FF, scale)
    rids, rw = oracle.route(lg, K, renorm, scale)
    assert np.array_equal(idr, rids) and same_bits(wr, rw)
    if case == "t80_e8":
        assert max(np.bincount(idr.reshape(-1))) > 12
    Y = g4.moe(ctx, wgu, wdn, X, rids, rw, D, FF)
    assert same_bits(Yr, Y)
    y64, bound = oracle.moe_exact(Q4_K, gu, Q4_K, dn, X, rids, rw, D, FF)
    for t in range(T):
        if t in bad:
            assert not np.any(np.isfinite(Y[t])), t
        else:
            assert_dots(Y[t], y64[t], bound[t], "moe grouped %s token %d" % (case, t))
    for t in (0, T - 1):
        Y1, _, _ = g4.moe_routed(ctx, wgu, wdn, X[t:t + 1], lg[t:t + 1], K, renorm, D, FF, scale)
        assert_dots(Y1[0], y64[t], bound[t], "moe token %d alone" % t)


def test_moe_routed_dev_calls(g4, ctx, oracle):
    """The device entry point on resident buffers, twice in a row with fewer tokens
    the second time: ids, weights and Y of each call match the host entry point."""
    import torch
    announce("moe routed dev calls")
    E, D, FF, K = 32, 256, 128, 4
    gu = synth.q4_k(55, "gu", E * 2 * FF * D)
    dn = synth.q4_k(55, "dn", E * D * FF)
    wgu = upload(g4, ctx, Q4_K, gu, E * 2 * FF * D)
    wdn = upload(g4, ctx, Q4_K, dn, E * D * FF)
    for call, T in enumerate([16, 3]):
        lg = synth.activations(55, "lg%d" % call, T * E).reshape(T, E)
        X = synth.activations(55, "X%d" % call, T * D).reshape(T, D)
        Yh, idh, wh = g4.moe_routed(ctx, wgu, wdn, X, lg, K, True, D, FF)
        d_ids = torch.full((T, K), -1, dtype=torch.int32, device="cuda")
        d_w = torch.zeros((T, K), dtype=torch.float32, device="cuda")
        d_Y = torch.zeros((T, D), dtype=torch.float32, device="cuda")
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        try:
            g4.moe_routed_dev(ctx, wgu, wdn, torch.from_numpy(X).cuda(), T, D, FF, torch.from_numpy(lg).cuda(), E,
                              K, True, d_ids.data_ptr(), d_w, d_Y)
            torch.cuda.synchronize()
        finally:
            ctx.set_stream(None)
        assert np.array_equal(d_ids.cpu().numpy(), idh), call
        assert same_bits(d_w.cpu().numpy(), wh), call
        assert same_bits(d_Y.cpu().numpy(), Yh), call


@pytest.mark.parametrize("case", ["one_expert", "widest_rows", "ragged_rows", "k8_e256"])
def test_moe_grouped_edges(g4, ctx, oracle, case):
    """Edges of the expert-grouped calls (41+ tokens) with the ids given:
    one_expert: all 256 pairs on one expert (16 passes of sixteen pairs, the other
    experts idle); widest_rows: 3072 columns, past the 16-pair tiles' 2048, so the
    eight-pair kernel (its largest LDS operand set, 150 KB); ragged_rows: rows of
    384 and 640 columns (3 and 5 of the 16 waves hold columns), down rows of 640
    columns (2.5 super-blocks, every second one staged from half way into one);
    k8_e256: 256 experts, eight slots per token."""
    announce("moe grouped edge %s" % case)
    E, D, FF, K, T = 16, 512, 256, 4, 64
    if case == "widest_rows":
        E, D, FF, K = 4, 3072, 128, 2
    elif case == "ragged_rows":
        D, FF = 384, 640
    elif case == "k8_e256":
        E, D, FF, K = 256, 256, 128, 8
    gu = synth.q4_k(62, "gu" + case, E * 2 * FF * D)
    dn = synth.q4_k(62, "dn" + case, E * D * FF)
    X = synth.activations(62, "X" + case, T * D).reshape(T, D)
    lg = synth.activations(62, "lg" + case, T * E).reshape(T, E)
    ids, gw = oracle.route(lg, K, True)
    if case == "one_expert":
        ids = np.full((T, K), 3, np.int32)
    wgu = upload(g4, ctx, Q4_K, gu, E * 2 * FF * D)
    wdn = upload(g4, ctx, Q4_K, dn, E * D * FF)
    Y = g4.moe(ctx, wgu, wdn, X, ids, gw, D, FF)
    y64, bound = oracle.moe_exact(Q4_K, gu, Q4_K, dn, X, ids, gw, D, FF)
    assert_dots(Y.reshape(-1), y64.reshape(-1), bound.reshape(-1), "moe grouped %s" % case)


@pytest.mark.parametrize("tokens", [1, 16, 64])
def test_moe_dev_out_of_range_ids(g4, ctx, oracle, tokens):
    """g4_moe_dev cannot check device ids: a pair whose id is outside [0, E) gets
    zero gate/up and down rows, so it adds w * 0 to its token's sum.  One token
    (down and weighted sum in one launch), 16 tokens (per-pair launches) and 64
    tokens (experts grouped on the matrix cores)."""
    import torch
    announce("moe dev out-of-range ids T=%d" % tokens)
    E, D, FF, K, T = 16, 512, 256, 4, tokens
    gu = synth.q4_k(59, "gu", E * 2 * FF * D)
    dn = synth.q4_k(59, "dn", E * D * FF)
    lg = synth.activations(59, "lg%d" % T, T * E).reshape(T, E)
    X = synth.activations(59, "X%d" % T, T * D).reshape(T, D)
    wgu = upload(g4, ctx, Q4_K, gu, E * 2 * FF * D)
    wdn = upload(g4, ctx, Q4_K, dn, E * D * FF)
    ids, gw = g4.moe_route(ctx, lg, K, True)
    bad = ids.copy()
    bad[0, 1] = -1
    bad[T - 1, K - 1] = E
    if T > 2:
        bad[T // 2, 0] = 1 << 30
    d_Y = torch.full((T, D), float("nan"), dtype=torch.float32, device="cuda")
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    try:
        g4.moe_dev(ctx, wgu, wdn, torch.from_numpy(X).cuda(), T, D, FF, torch.from_numpy(bad).cuda(),
                   torch.from_numpy(gw).cuda(), K, d_Y)
        torch.cuda.synchronize()
    finally:
        ctx.set_stream(None)
    Y = d_Y.cpu().numpy()
    # the oracle with those slots' weights zeroed (their ids made valid)
    ids0, w0 = bad.copy(), gw.copy()
    off = (bad < 0) | (bad >= E)
    ids0[off] = 0
    w0[off] = 0.0
    y64, bound = oracle.moe_exact(Q4_K, gu, Q4_K, dn, X, ids0, w0, D, FF)
    assert_dots(Y.reshape(-1), y64.reshape(-1), bound.reshape(-1), "moe dev bad ids T=%d" % T)


def test_moe_repeated_calls(g4, ctx, oracle):
    """Back-to-back MoE calls on one context with changing token counts: the
    context's scratch is re-carved per call and nothing leaks from one call to the next.
    41 and 48 tokens run the experts grouped; 25, 31 and 33 take the per-pair
    launches with pair counts (100, 124, 132) that do not divide the resident
    workgroups."""
    announce("moe repeated calls")
    E, D, FF, K = 16, 512, 256, 4
    gu = synth.q4_k(48, "gu", E * 2 * FF * D)
    dn = synth.q4_k(48, "dn", E * D * FF)
    wgu = upload(g4, ctx, Q4_K, gu, E * 2 * FF * D)
    wdn = upload(g4, ctx, Q4_K, dn, E * D * FF)
    for call, T in enumerate([3, 16, 1, 16, 48, 2, 31, 25, 33, 41]):
        lg = synth.activations(48, "lg%d" % call, T * E).reshape(T, E)
        X = synth.activations(48, "X%d" % call, T * D).reshape(T, D)
        ids, gw = g4.moe_route(ctx, lg, K, True)
        Y = g4.moe(ctx, wgu, wdn, X, ids, gw, D, FF)
        y64, bound = oracle.moe_exact(Q4_K, gu, Q4_K, dn, X, ids, gw, D, FF)
        assert_dots(Y.reshape(-1), y64.reshape(-1), bound.reshape(-1), "call %d T=%d" % (call, T))


def test_moe_reference_gates(g4, ctx, oracle):
    """Un-renormalised gates times a per-expert down scale, as Llama.kt:300-337 uses them."""
    announce("moe reference gates")
    E, D, FF, K, T = 16, 512, 256, 4, 3
    gu = synth.q8_0(47, "gu", E * 2 * FF * D)
    dn = synth.q8_0(47, "dn", E * D * FF)
    lg = synth.activations(47, "lg", T * E).reshape(T, E)
    X = synth.activations(47, "X", T * D).reshape(T, D)
    scale = np.linspace(0.25, 2.0, E).astype(np.float32)
    wgu = upload(g4, ctx, Q8_0, gu, E * 2 * FF * D)
    wdn = upload(g4, ctx, Q8_0, dn, E * D * FF)
    ids, gw = g4.moe_route(ctx, lg, K, False, scale)
    Y = g4.moe(ctx, wgu, wdn, X, ids, gw, D, FF)
    y64, bound = oracle.moe_exact(Q8_0, gu, Q8_0, dn, X, ids, gw, D, FF)
    assert_dots(Y.reshape(-1), y64.reshape(-1), bound.reshape(-1), "moe ref gates")
    y32 = oracle.moe(Q8_0, gu, Q8_0, dn, X, ids, gw, D, FF)
    assert_dots(y32.reshape(-1), y64.reshape(-1), bound.reshape(-1), "oracle moe")


# ------------------------------------------------------------------ argmax ---

@pytest.mark.parametrize("case", ["ties", "nan_first", "nan_later", "neg_inf", "signed_zero", "random_big"])
def test_argmax_cases(g4, ctx, oracle, case):
    announce("argmax %s" % case)
    rng = np.random.default_rng(8)
    v = rng.standard_normal(300000).astype(np.float32)
    if case == "ties":
        v[1234] = v[99999] = v[250000] = 50.0
    elif case == "nan_first":
        v[0] = np.nan
        v[7] = 100.0
    elif case == "nan_later":
        v[5] = np.nan
        v[200000] = 60.0
    elif case == "neg_inf":
        v[:] = -np.inf
    elif case == "signed_zero":
        v[:] = -1.0
        v[1000] = -0.0
        v[2000] = 0.0
    assert g4.argmax(ctx, v) == oracle.argmax(v)


@pytest.mark.parametrize("case", ["ties", "zeros", "nan", "e100", "e300", "e1024", "k_all"])
def test_moe_route_edge_cases(g4, ctx, oracle, case):
    """Top-k ties (lowest index first), probabilities that underflow to 0, a NaN
    logit (the scans keep index 0 once nothing beats -inf), expert counts that are
    not a multiple of the workgroup, and k = n_experts."""
    announce("moe route %s" % case)
    rng = np.random.default_rng(49)
    E, K, T = 128, 8, 3
    if case == "e100":
        E = 100
    elif case == "e300":
        E = 300
    elif case == "e1024":
        E, K = 1024, 16
    elif case == "k_all":
        E, K = 64, 64
    lg = rng.standard_normal((T, E)).astype(np.float32)
    if case == "ties":
        lg[:, :] = np.round(lg * 2) / 2      # many equal logits
        lg[0, :] = 1.0                        # every logit equal
    elif case == "zeros":
        lg[:, :] = -1000.0                    # exp underflows to 0 except the maximum
        lg[:, 5] = 0.0
        lg[1, 70] = 0.0
    elif case == "nan":
        lg[1, 17] = np.nan
    for renorm in (True, False):
        ids, w = g4.moe_route(ctx, lg, K, renorm)
        rids, rw = oracle.route(lg, K, renorm)
        assert np.array_equal(ids, rids), (case, renorm)
        assert same_bits(w, rw), (case, renorm)
