"""GPU parity of the decode-step entry points of libg4hip.so against the CPU
oracle: rms norm (Llama.kt:27-78), residual add (MutableFloatTensor.kt:28-37),
logit soft-capping (Llama.kt:403-406), the norm fused into the matvec, the dense
FFN block (Llama.kt:355-363) and the LM-head tail (Llama.kt:401-407 + argmax).

Bars (written into each check):
  * rms norm: bit-exact against the oracle's restatement on integer inputs,
    whose sum of squares is exact in any order (so the scale is fixed and each
    form's product order is checked); |y - exact| <= 1e-5 |exact| against the fp64
    norm on random inputs (the summation order differs from the reference's
    sequential one);
  * residual add: bit-exact;
  * soft-capping: within 2 ulp of cap * tanh(v / cap) evaluated in fp64 (the
    reference rounds a double tanh to float; the oracle and the device both run
    fdlibm's tanh, over the C library's and the device's own expm1, which may
    differ in a last double bit);
  * norm fused into the matvec: bit-identical to the standalone norm followed by
    the plain matvec, and every dot within 1e-5 * sum |w_i xn_i|;
  * blocks: within the error bound the fp64 oracle carries through the block
    (or_ffn_block_exact / or_lm_head_exact: 1e-5 per norm scale and per dot);
    the LM head's argmax exact, with the top-1/top-2 gap checked.
"""
import numpy as np
import pytest

import synth
from conftest import announce

pytestmark = pytest.mark.gpu

Q8_0, Q4_0, Q4_K, Q5_K, Q6_K, F16, BF16, F32 = 8, 2, 12, 13, 14, 1, 30, 0
TOL = 1e-5


def same_bits(a, b) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn]))


def within(y, exact, bound, what=""):
    y = np.asarray(y, np.float64)
    err = np.abs(y - exact)
    bad = np.nonzero(err > bound)[0]
    assert bad.size == 0, "%s: %d values out of tolerance, first %d: y=%r exact=%r bound=%r" % (
        what, bad.size, bad[0], y[bad[0]], exact[bad[0]], bound[bad[0]])


def upload(g4, ctx, t, raw, n):
    return g4.FloatTensorFactory.create(ctx, t, raw, n)


def upload_norm(g4, ctx, w):
    return upload(g4, ctx, F32, np.ascontiguousarray(w, np.float32), w.size)


@pytest.fixture
def dev(ctx):
    """Run the context's *_dev calls on torch's current stream; yields torch."""
    import torch
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    try:
        yield torch
    finally:
        torch.cuda.synchronize()
        ctx.set_stream(None)


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def host(torch, t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


# ----------------------------------------------------------------- rmsnorm ---

NORM_CASES = [(1, 2048), (8, 256), (3, 999), (1, 1), (2, 5376)]


@pytest.mark.parametrize("form", [0, 1, 2])
@pytest.mark.parametrize("n_vec,size", NORM_CASES)
def test_rmsnorm_exact_sum_bit_exact(g4, ctx, oracle, dev, form, n_vec, size):
    announce("rmsnorm exact-sum form=%d n_vec=%d size=%d" % (form, n_vec, size))
    rng = np.random.default_rng(100 + size)
    x = rng.integers(-64, 65, (n_vec, size)).astype(np.float32)
    w = (1 + 0.25 * rng.standard_normal(size)).astype(np.float32)
    wt = upload_norm(g4, ctx, w) if form != 2 else None
    xd = to_dev(dev, x)
    out = dev.empty_like(xd)
    g4.rmsnorm_dev(ctx, wt, xd, out, n_vec, size, 1e-6, form)
    got = host(dev, out)
    want = np.stack([oracle.rmsnorm(x[v], w if form != 2 else None, 1e-6, form) for v in range(n_vec)])
    assert same_bits(got, want)
    # in place gives the same bits
    g4.rmsnorm_dev(ctx, wt, xd, xd, n_vec, size, 1e-6, form)
    assert same_bits(host(dev, xd), want)


@pytest.mark.parametrize("eps", [1e-6, 0.1])
@pytest.mark.parametrize("n_vec,size", NORM_CASES)
def test_rmsnorm_random_vs_fp64(g4, ctx, oracle, dev, eps, n_vec, size):
    announce("rmsnorm random eps=%g n_vec=%d size=%d" % (eps, n_vec, size))
    x = synth.activations(101, "nx%d" % size, n_vec * size, 3.0).reshape(n_vec, size)
    w = synth.norm_weight(101, "nw%d" % size, size)
    wt = upload_norm(g4, ctx, w)
    xd = to_dev(dev, x)
    for form in (0, 1, 2):
        out = dev.empty_like(xd)
        g4.rmsnorm_dev(ctx, wt if form != 2 else None, xd, out, n_vec, size, eps, form)
        got = host(dev, out)
        for v in range(n_vec):
            ex = oracle.rmsnorm_exact(x[v], w if form != 2 else None, eps)
            within(got[v], ex, TOL * np.abs(ex) + 1e-30, "form %d vec %d" % (form, v))


def test_rmsnorm_add(g4, ctx, oracle, dev):
    announce("rmsnorm_add")
    size = 2048
    rng = np.random.default_rng(102)
    v = rng.integers(-64, 65, size).astype(np.float32)
    x = synth.activations(102, "x", size, 4.0)
    w = synth.norm_weight(102, "w", size)
    wt = upload_norm(g4, ctx, w)
    vd, xd = to_dev(dev, v), to_dev(dev, x)
    g4.rmsnorm_add_dev(ctx, wt, vd, xd, size, 1e-6)
    vn = oracle.rmsnorm(v, w, 1e-6)
    assert same_bits(host(dev, vd), vn)
    assert same_bits(host(dev, xd), x + vn)


def test_add_bit_exact(g4, ctx, dev):
    announce("add")
    a = synth.activations(103, "a", 100003)
    b = synth.activations(103, "b", 100003, 1e-3)
    ad, bd = to_dev(dev, a), to_dev(dev, b)
    g4.add_dev(ctx, ad, bd, a.size)
    assert same_bits(host(dev, ad), a + b)


def test_softcap(g4, ctx, oracle, dev):
    announce("softcap")
    cap = 30.0
    v = np.concatenate([synth.activations(104, "v", 200000, 20.0),
                        np.array([0.0, -0.0, 1e-30, 1e9, -1e9, np.inf, -np.inf, np.nan], np.float32)])
    vd = to_dev(dev, v)
    g4.softcap_dev(ctx, vd, v.size, cap)
    got = host(dev, vd)
    fin = np.isfinite(v)
    ref = (cap * np.tanh(v[fin].astype(np.float64) / cap)).astype(np.float32)
    ulp = np.spacing(np.abs(ref))
    assert np.all(np.abs(got[fin].astype(np.float64) - ref) <= 2 * ulp)
    assert same_bits(got[~fin], oracle.softcap(v[~fin], cap))
    # the oracle and the device agree except, rarely, in the last bit (expm1)
    orc = oracle.softcap(v, cap)
    assert np.count_nonzero(got[fin] != orc[fin]) <= v.size // 10000


# ------------------------------------------------- norm fused in the matvec ---

FUSED = [
    # (type, dim0, dim1, row offset): 16/32/64-lane groups, two chunks per lane,
    # several column passes (standalone norm), rows off the 64-element grid (generic)
    (Q8_0, 96, 640, 0), (Q4_0, 96, 2048, 1), (Q4_K, 64, 2560, 0), (Q6_K, 48, 5376, 0),
    (F16, 40, 2048, 0), (Q8_0, 24, 16384, 0), (F32, 7, 1000, 0)]


@pytest.mark.parametrize("t,dim0,dim1,roff", FUSED, ids=[str(f) for f in FUSED])
def test_matmul_norm_fused_equals_unfused(g4, ctx, oracle, dev, t, dim0, dim1, roff):
    announce("matmul_norm type=%d dim0=%d dim1=%d roff=%d" % (t, dim0, dim1, roff))
    n = (dim0 + roff) * dim1
    n = (n + 255) // 256 * 256
    raw = synth.weights(105, "mn%d.%d" % (t, dim1), t, n)
    x = synth.activations(105, "mnx%d" % dim1, dim1, 3.0)
    nw = synth.norm_weight(105, "mnw%d" % dim1, dim1)
    w = upload(g4, ctx, t, raw, n)
    nt = upload_norm(g4, ctx, nw)
    off = roff * dim1
    xd = to_dev(dev, x)
    out = dev.empty(dim0, dtype=dev.float32, device="cuda")
    xn = dev.empty(dim1, dtype=dev.float32, device="cuda")
    g4.matmul_norm_dev(ctx, w, nt, xd, out, dim0, dim1, 1e-6, off, xnorm=xn)
    fused, fused_xn = host(dev, out), host(dev, xn)
    # the same without xnorm output
    out2 = dev.empty(dim0, dtype=dev.float32, device="cuda")
    g4.matmul_norm_dev(ctx, w, nt, xd, out2, dim0, dim1, 1e-6, off)
    # standalone norm, then the plain matvec
    xs = dev.empty(dim1, dtype=dev.float32, device="cuda")
    g4.rmsnorm_dev(ctx, nt, xd, xs, 1, dim1, 1e-6, 0)
    out3 = dev.empty(dim0, dtype=dev.float32, device="cuda")
    w.matmul_dev(xs, out3, dim0, dim1, off)
    xs_h = host(dev, xs)
    assert same_bits(fused_xn, xs_h)
    assert same_bits(fused, host(dev, out3))
    assert same_bits(host(dev, out2), fused)
    exn = oracle.rmsnorm_exact(x, nw, 1e-6)
    within(xs_h, exn, TOL * np.abs(exn) + 1e-30, "norm")
    ex, ab = oracle.matmul_exact(t, raw, xs_h, dim0, dim1, off)
    within(fused, ex, TOL * ab + 1e-30, "dots")


# --------------------------------------------------------------- FFN block ---

def _ffn_block_check(g4, ctx, oracle, tg, tu, td, gate, up, down, npre, npost, x, dim, hidden, eps, what):
    wg = upload(g4, ctx, tg, gate, hidden * dim)
    wu = upload(g4, ctx, tu, up, hidden * dim)
    wd = upload(g4, ctx, td, down, dim * hidden)
    n1, n2 = upload_norm(g4, ctx, npre), upload_norm(g4, ctx, npost)
    got = g4.ffn_block(ctx, wg, wu, wd, n1, n2, x, dim, hidden, eps)
    x64, b64 = oracle.ffn_block_exact(tg, gate, tu, up, td, down, npre, npost, x, dim, hidden, eps)
    within(got, x64, TOL * b64, what)
    ref = oracle.ffn_block(tg, gate, tu, up, td, down, npre, npost, x, dim, hidden, eps)
    within(ref, x64, TOL * b64, what + " (oracle restatement)")
    return (wg, wu, wd, n1, n2), got


def test_ffn_block_q4_0_workload(g4, ctx, oracle, dev):
    announce("workload q4_0 ffn block 8192x2048 + norms + residual")
    c = synth.q4_0_ffn_block()
    dim, hidden, eps = c["dim"], c["hidden"], c["eps"]
    ws, got = _ffn_block_check(g4, ctx, oracle, Q4_0, Q4_0, Q4_0, c["gate"], c["up"], c["down"], c["norm_pre"],
                               c["norm_post"], c["x"], dim, hidden, eps, "ffn block")
    # the device form, twice in a row (x is updated in place each time)
    xd = to_dev(dev, c["x"])
    g4.ffn_block_dev(ctx, *ws, xd, dim, hidden, eps)
    assert same_bits(host(dev, xd), got)
    g4.ffn_block_dev(ctx, *ws, xd, dim, hidden, eps)
    again = g4.ffn_block(ctx, *ws, got, dim, hidden, eps)
    assert same_bits(host(dev, xd), again)


@pytest.mark.parametrize("tg,td,dim,hidden", [(Q4_K, Q6_K, 1024, 2816), (Q8_0, Q8_0, 640, 1536),
                                              (Q5_K, Q4_K, 2560, 1024), (F32, F32, 1000, 300)])
def test_ffn_block_formats(g4, ctx, oracle, tg, td, dim, hidden):
    announce("ffn block gate/up=%d down=%d dim=%d hidden=%d" % (tg, td, dim, hidden))
    gate = synth.weights(106, "g%d" % dim, tg, hidden * dim)
    up = synth.weights(106, "u%d" % dim, tg, hidden * dim)
    down = synth.weights(106, "d%d" % dim, td, dim * hidden)
    npre, npost = synth.norm_weight(106, "a%d" % dim, dim), synth.norm_weight(106, "b%d" % dim, dim)
    x = synth.activations(106, "x%d" % dim, dim, 4.0)
    _ffn_block_check(g4, ctx, oracle, tg, tg, td, gate, up, down, npre, npost, x, dim, hidden, 1e-6,
                     "ffn block %d/%d" % (tg, td))


# ----------------------------------------------------------------- LM head ---

def _lm_check(logits, idx, l64, b64, what):
    within(logits, l64, TOL * b64, what)
    order = np.argsort(-l64, kind="stable")
    gap = l64[order[0]] - l64[order[1]]
    assert gap > TOL * (b64[order[0]] + b64[order[1]]), "%s: fixture gap too small to pin the argmax" % what
    assert idx == int(order[0])


def test_lm_head_softcap_workload(g4, ctx, oracle, dev):
    announce("workload q8_0 lm head 262144x2048 + final norm + softcap 30 + argmax")
    c = synth.q8_0_lm_head_block()
    V, D, eps, cap = c["dim0"], c["dim1"], c["eps"], c["cap"]
    w = upload(g4, ctx, Q8_0, c["w"], V * D)
    nt = upload_norm(g4, ctx, c["norm"])
    logits, idx = g4.lm_head(ctx, w, nt, c["x"], V, D, eps, cap)
    l64, b64 = oracle.lm_head_exact(Q8_0, c["w"], c["norm"], c["x"], V, D, eps, cap)
    _lm_check(logits, idx, l64, b64, "lm head")
    assert idx == oracle.argmax(logits)
    assert np.all(np.abs(logits) <= cap)
    # index only, and the device form with the normalised x
    assert g4.lm_head(ctx, w, nt, c["x"], V, D, eps, cap, want_logits=False)[1] == idx
    xd = to_dev(dev, c["x"])
    xn = dev.empty(D, dtype=dev.float32, device="cuda")
    ld = dev.empty(V, dtype=dev.float32, device="cuda")
    ix = dev.zeros(1, dtype=dev.int32, device="cuda")
    g4.lm_head_dev(ctx, w, nt, xd, ld, ix, V, D, eps, cap, xnorm=xn)
    assert int(host(dev, ix)[0]) == idx
    assert same_bits(host(dev, ld), logits)
    xs = dev.empty(D, dtype=dev.float32, device="cuda")
    g4.rmsnorm_dev(ctx, nt, xd, xs, 1, D, eps, 0)
    assert same_bits(host(dev, xn), host(dev, xs))


@pytest.mark.parametrize("cap", [0.0, 30.0])
@pytest.mark.parametrize("t,vocab,dim", [(Q8_0, 50000, 2048), (Q4_K, 30000, 2560), (Q8_0, 4000, 16384),
                                         (F16, 3000, 1000)])
def test_lm_head_shapes(g4, ctx, oracle, cap, t, vocab, dim):
    announce("lm head type=%d vocab=%d dim=%d cap=%g" % (t, vocab, dim, cap))
    raw = synth.weights(107, "lm%d.%d" % (t, dim), t, vocab * dim)
    nw = synth.norm_weight(107, "ln%d" % dim, dim, 0.05)  # logits well below the cap (no saturated ties)
    x = synth.activations(107, "lx%d" % dim, dim)
    w = upload(g4, ctx, t, raw, vocab * dim)
    nt = upload_norm(g4, ctx, nw)
    logits, idx = g4.lm_head(ctx, w, nt, x, vocab, dim, 1e-6, cap)
    l64, b64 = oracle.lm_head_exact(t, raw, nw, x, vocab, dim, 1e-6, cap)
    _lm_check(logits, idx, l64, b64, "lm head %d" % t)
    assert idx == oracle.argmax(logits)


# ------------------------------------------------------------------ errors ---

def test_step_errors(g4, ctx, dev):
    announce("decode-step errors")
    dim = 256
    w = upload(g4, ctx, Q8_0, synth.q8_0(108, "w", 64 * dim), 64 * dim)
    n16 = upload(g4, ctx, F16, synth.dense(108, "n", dim, F16), dim)
    nshort = upload_norm(g4, ctx, np.ones(dim // 2, np.float32))
    nt = upload_norm(g4, ctx, np.ones(dim, np.float32))
    x = np.ones(dim, np.float32)
    with pytest.raises(g4.UnsupportedOperationException):
        g4.lm_head(ctx, w, n16, x, 64, dim, 1e-6, 30.0)
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.lm_head(ctx, w, nshort, x, 64, dim, 1e-6, 30.0)
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.lm_head(ctx, w, nt, x, 65, dim, 1e-6, 30.0)
    with pytest.raises(g4.IllegalArgumentException):
        g4.lm_head(ctx, w, nt, x, 64, dim, float("nan"), 30.0)
    xd = to_dev(dev, x)
    with pytest.raises(g4.IllegalArgumentException):
        g4.softcap_dev(ctx, xd, dim, 0.0)
    with pytest.raises(g4.IllegalArgumentException):
        g4.rmsnorm_dev(ctx, nt, xd, xd, 1, dim, 1e-6, 3)
    with pytest.raises(g4.IllegalArgumentException):
        g4.rmsnorm_add_dev(ctx, nt, xd, xd, dim, 1e-6)
    out = dev.empty(64, dtype=dev.float32, device="cuda")
    with pytest.raises(g4.IllegalArgumentException):
        g4.matmul_norm_dev(ctx, w, nt, xd, out, 64, dim, 1e-6, xnorm=xd)


# ------------------------------------------------------------ load hook ---

def test_blocks_from_a_gguf_file(g4, ctx, oracle, tmp_path):
    """The load hook end to end: tensors written to a GGUF file, parsed and mapped
    (gguf.GGUF, GGUF.kt:195-212), uploaded through ModelLoader.load_quantized
    (ModelLoader.kt:268-271 -> FloatTensorFactory.create), then the dense FFN block
    and the LM-head tail run on the uploaded tensors with the file's eps and cap."""
    import gguf
    from gguf_writer import FLOAT32, STRING, write_gguf
    announce("gguf load hook: ffn block + lm head from a file")
    dim, hidden, vocab = 1024, 2816, 8192
    src = {
        "blk.0.ffn_gate.weight": ((dim, hidden), Q4_K, synth.q4_k(109, "g", hidden * dim)),
        "blk.0.ffn_up.weight": ((dim, hidden), Q4_K, synth.q4_k(109, "u", hidden * dim)),
        "blk.0.ffn_down.weight": ((hidden, dim), Q6_K, synth.q6_k(109, "d", dim * hidden)),
        "blk.0.ffn_norm.weight": ((dim,), F32, synth.norm_weight(109, "n1", dim)),
        "blk.0.post_ffw_norm.weight": ((dim,), F32, synth.norm_weight(109, "n2", dim)),
        "output_norm.weight": ((dim,), F32, synth.norm_weight(109, "n3", dim, 0.05)),
        "token_embd.weight": ((dim, vocab), Q8_0, synth.q8_0(109, "e", vocab * dim)),
    }
    path = str(tmp_path / "model.gguf")
    write_gguf(path, [("general.architecture", STRING, "gemma4"),
                      ("gemma4.attention.layer_norm_rms_epsilon", FLOAT32, 1e-6),
                      ("gemma4.final_logit_softcapping", FLOAT32, 30.0)],
               [(n, d, t, raw) for n, (d, t, raw) in src.items()], alignment=64)
    g = gguf.GGUF.load_model(path)
    entries = gguf.GGUF.load_tensors(path, g.tensor_data_offset, g.tensor_infos)
    dv = {n: gguf.ModelLoader.load_quantized(ctx, e) for n, e in entries.items()}
    eps = g.metadata["gemma4.attention.layer_norm_rms_epsilon"]
    cap = g.metadata["gemma4.final_logit_softcapping"]
    for n, (d, t, raw) in src.items():
        assert dv[n].size == int(np.prod(d)) and dv[n].nbytes == raw.nbytes
    r = {n: raw for n, (d, t, raw) in src.items()}
    x = synth.activations(109, "x", dim, 4.0)
    x1 = g4.ffn_block(ctx, dv["blk.0.ffn_gate.weight"], dv["blk.0.ffn_up.weight"], dv["blk.0.ffn_down.weight"],
                      dv["blk.0.ffn_norm.weight"], dv["blk.0.post_ffw_norm.weight"], x, dim, hidden, eps)
    x64, b64 = oracle.ffn_block_exact(Q4_K, r["blk.0.ffn_gate.weight"], Q4_K, r["blk.0.ffn_up.weight"], Q6_K,
                                      r["blk.0.ffn_down.weight"], r["blk.0.ffn_norm.weight"],
                                      r["blk.0.post_ffw_norm.weight"], x, dim, hidden, eps)
    within(x1, x64, TOL * b64, "ffn block from gguf")
    logits, idx = g4.lm_head(ctx, dv["token_embd.weight"], dv["output_norm.weight"], x1, vocab, dim, eps, cap)
    l64, lb = oracle.lm_head_exact(Q8_0, r["token_embd.weight"], r["output_norm.weight"], x1, vocab, dim, eps, cap)
    _lm_check(logits, idx, l64, lb, "lm head from gguf")
