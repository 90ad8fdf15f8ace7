"""GPU parity of g4_attention_dev (decode attention over a KV cache,
Llama.kt:198-218) against the CPU oracle.

Bar: |out - exact| <= 1e-5 * bound (or_attention_exact: each score may be off by
1e-5 of its sum |q k|, which moves each softmax weight by at most twice that of
itself; plus rounding of the weighted sums), and the oracle's restatement meets the
same bound.  A single position returns its V row bit-exactly (exp(0) = 1)."""
import numpy as np
import pytest

import synth
from conftest import announce

pytestmark = pytest.mark.gpu


def same_bits(a, b) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))


def _inputs(seed, n_heads, n_kv, hs, rows):
    q = synth.activations(seed, "q", n_heads * hs)
    kc = synth.activations(seed, "k", rows * n_kv * hs)
    vc = synth.activations(seed, "v", rows * n_kv * hs)
    return q, kc, vc


def _run(g4, ctx, torch, q, kc, vc, n_heads, n_kv, hs, position, start, shift=0):
    """shift > 0 offsets every device buffer by that many floats (unaligned pointers)."""
    def dev(a):
        t = torch.zeros(a.size + shift, dtype=torch.float32, device="cuda")
        t[shift:] = torch.from_numpy(np.ascontiguousarray(a))
        return t, t[shift:]
    _, qd = dev(q)
    _, kd = dev(kc)
    _, vd = dev(vc)
    ob, od = dev(np.zeros(n_heads * hs, np.float32))
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    try:
        g4.attention_dev(ctx, qd, kd, vd, od, n_heads, n_kv, hs, position, start)
        torch.cuda.synchronize()
    finally:
        ctx.set_stream(None)
    return od.cpu().numpy().reshape(n_heads, hs)


CASES = [
    # (n_heads, n_kv, head_size, position, att_start)
    (16, 8, 256, 8191, 0),    # long context, kv_mul 2
    (8, 2, 256, 4095, 0),     # kv_mul 4
    (8, 1, 128, 1000, 489),   # sliding window of 512
    (4, 4, 64, 77, 0),        # no sharing, short
    (8, 1, 512, 300, 0),      # head size 512, kv_mul 8: two head groups
    (6, 2, 256, 200, 0),      # kv_mul 3: a partly filled head group
    (4, 2, 80, 50, 0),        # head size 80: one workgroup per head
    (2, 1, 256, 20000, 19000),
]


@pytest.mark.parametrize("n_heads,n_kv,hs,position,start", CASES, ids=[str(c) for c in CASES])
def test_attention_vs_fp64(g4, ctx, oracle, n_heads, n_kv, hs, position, start):
    import torch
    announce("attention heads=%d kv=%d hs=%d pos=%d start=%d" % (n_heads, n_kv, hs, position, start))
    q, kc, vc = _inputs(110 + hs, n_heads, n_kv, hs, position + 1)
    out = _run(g4, ctx, torch, q, kc, vc, n_heads, n_kv, hs, position, start)
    o64, b64 = oracle.attention_exact(q, kc, vc, n_heads, n_kv, hs, position, start)
    err = np.abs(out.astype(np.float64) - o64)
    assert np.all(err <= 1e-5 * b64), "max err %g at bound %g" % (err.max(), (1e-5 * b64).ravel()[err.argmax()])
    # tighter than the bound in practice: report-level check on the typical error
    assert np.max(err / (np.abs(o64) + 1e-3)) < 1e-3
    if position - start < 5000:
        ref = oracle.attention(q, kc, vc, n_heads, n_kv, hs, position, start)
        assert np.all(np.abs(ref - o64) <= 1e-5 * b64)


def test_attention_single_position_is_v(g4, ctx):
    import torch
    announce("attention single position")
    n_heads, n_kv, hs = 8, 2, 256
    q, kc, vc = _inputs(111, n_heads, n_kv, hs, 1)
    out = _run(g4, ctx, torch, q, kc, vc, n_heads, n_kv, hs, 0, 0)
    v = vc.reshape(n_kv, hs)
    assert same_bits(out, np.repeat(v, n_heads // n_kv, axis=0))


def test_attention_window_never_reads_before_start(g4, ctx, oracle):
    import torch
    announce("attention window rows")
    n_heads, n_kv, hs, position, start = 4, 2, 256, 700, 600
    q, kc, vc = _inputs(112, n_heads, n_kv, hs, position + 1)
    kc.reshape(position + 1, -1)[:start] = np.nan
    vc.reshape(position + 1, -1)[:start] = np.nan
    out = _run(g4, ctx, torch, q, kc, vc, n_heads, n_kv, hs, position, start)
    assert np.all(np.isfinite(out))
    o64, b64 = oracle.attention_exact(q, kc, vc, n_heads, n_kv, hs, position, start)
    assert np.all(np.abs(out - o64) <= 1e-5 * b64)


def test_attention_unaligned_buffers(g4, ctx, oracle):
    import torch
    announce("attention unaligned buffers")
    n_heads, n_kv, hs, position = 4, 2, 256, 129
    q, kc, vc = _inputs(113, n_heads, n_kv, hs, position + 1)
    out = _run(g4, ctx, torch, q, kc, vc, n_heads, n_kv, hs, position, 0, shift=1)
    o64, b64 = oracle.attention_exact(q, kc, vc, n_heads, n_kv, hs, position, 0)
    assert np.all(np.abs(out - o64) <= 1e-5 * b64)


def test_attention_errors(g4, ctx):
    import torch
    announce("attention errors")
    t = torch.zeros(4096, dtype=torch.float32, device="cuda")
    with pytest.raises(g4.IllegalArgumentException):
        g4.attention_dev(ctx, t, t, t, t, 6, 4, 64, 3, 0)   # heads not a multiple of kv heads
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.attention_dev(ctx, t, t, t, t, 4, 2, 64, 3, 5)   # start past position
    with pytest.raises(g4.IllegalArgumentException):
        g4.attention_dev(ctx, t, t, t, t, 4, 2, 0, 3, 0)
