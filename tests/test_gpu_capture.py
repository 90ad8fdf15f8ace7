"""HIP graph capture over the device-pointer entry points.

A graph keeps the device addresses it was recorded with, including the
context's scratch (MoE hidden vectors and per-slot outputs here).  The library
therefore (1) refuses to grow the scratch while the stream is capturing,
recording nothing, (2) after a capture keeps an outgrown scratch buffer alive
instead of freeing it, so earlier graphs still replay into valid memory, and (3)
refuses host-pointer calls, which synchronise, under capture.  Every replay is
compared with the eager result, with eager work and synchronisation between
replays."""
import numpy as np
import pytest
import torch

import synth
from conftest import announce

pytestmark = pytest.mark.gpu

Q4_K = 12


@pytest.fixture(scope="module")
def moe_weights(g4, ctx):
    E, dim, ff = 16, 512, 256
    gu = synth.q4_k(41, "gu", E * 2 * ff * dim)
    dn = synth.q4_k(41, "dn", E * dim * ff)
    wgu = g4.FloatTensorFactory.create(ctx, Q4_K, gu, E * 2 * ff * dim)
    wdn = g4.FloatTensorFactory.create(ctx, Q4_K, dn, E * dim * ff)
    yield dict(E=E, dim=dim, ff=ff, k=4, wgu=wgu, wdn=wdn)
    wgu.free()
    wdn.free()


@pytest.fixture(scope="module")
def wide_moe_weights(g4, ctx):
    """The configured expert shape (dim 2048, ff 1408): its grouped launches need
    about 98 KB (gate+up) and 67 KB (down) of LDS, more than the 64 KB a kernel
    gets without its attribute."""
    E, dim, ff = 8, 2048, 1408
    gu = synth.q4_k(42, "gu", E * 2 * ff * dim)
    dn = synth.q4_k(42, "dn", E * dim * ff)
    wgu = g4.FloatTensorFactory.create(ctx, Q4_K, gu, E * 2 * ff * dim)
    wdn = g4.FloatTensorFactory.create(ctx, Q4_K, dn, E * dim * ff)
    yield dict(E=E, dim=dim, ff=ff, k=4, wgu=wgu, wdn=wdn)
    wgu.free()
    wdn.free()


def _io(mw, T, seed):
    X = torch.from_numpy(synth.activations(seed, "x", T * mw["dim"]).reshape(T, mw["dim"])).cuda()
    lg = torch.from_numpy(synth.activations(seed, "lg", T * mw["E"]).reshape(T, mw["E"])).cuda()
    ids = torch.zeros((T, mw["k"]), dtype=torch.int32, device="cuda")
    w = torch.zeros((T, mw["k"]), dtype=torch.float32, device="cuda")
    Y = torch.empty((T, mw["dim"]), dtype=torch.float32, device="cuda")
    return X, lg, ids, w, Y


def _moe(g4, c, mw, T, io):
    X, lg, ids, w, Y = io
    g4.moe_routed_dev(c, mw["wgu"], mw["wdn"], X, T, mw["dim"], mw["ff"], lg, mw["E"], mw["k"], True, ids, w, Y)


def _capture(c, stream, fn):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        c.set_stream(stream.cuda_stream)
        fn()
    c.set_stream(None)
    return g


def test_replays_survive_a_later_scratch_regrowth(g4, moe_weights):
    announce("capture: replay after the scratch regrows")
    mw = moe_weights
    c = g4.Context(0)
    stream = torch.cuda.Stream()
    try:
        small = _io(mw, 4, 1)
        _moe(g4, c, mw, 4, small)  # eager: sizes the scratch for 4 tokens
        torch.cuda.synchronize()
        want = small[4].clone()
        before = c.scratch_bytes()
        small[4].fill_(float("nan"))
        g = _capture(c, stream, lambda: _moe(g4, c, mw, 4, small))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(small[4], want)
        # a larger eager call outgrows the scratch the graph recorded
        big = _io(mw, 96, 2)
        _moe(g4, c, mw, 96, big)
        torch.cuda.synchronize()
        assert c.scratch_bytes() > before
        Y_big = big[4].clone()
        for rep in range(3):
            small[4].fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(small[4], want), "replay %d" % rep
            # eager work on the new scratch between replays stays correct too
            _moe(g4, c, mw, 96, big)
            torch.cuda.synchronize()
            assert torch.equal(big[4], Y_big)
    finally:
        torch.cuda.synchronize()
        c.close()


@pytest.mark.parametrize("shape", ["dim512", "dim2048_ff1408"])
def test_grouped_moe_replays(g4, request, shape):
    """A call of 96 tokens runs the experts grouped by expert: a routing launch, two
    grouped launches and the combine.  At dim 2048 / ff 1408 the grouped kernels
    use more than 64 KB of LDS (granted once per device when the context opens,
    never inside a capture).  Captured once and replayed three times, with eager
    grouped and per-pair calls between the replays: every replay gives the eager
    bits."""
    announce("capture: grouped MoE replays %s" % shape)
    mw = request.getfixturevalue("moe_weights" if shape == "dim512" else "wide_moe_weights")
    c = g4.Context(0)
    stream = torch.cuda.Stream()
    try:
        big = _io(mw, 96, 5)
        small = _io(mw, 4, 6)
        _moe(g4, c, mw, 96, big)  # eager: sizes the scratch
        _moe(g4, c, mw, 4, small)
        torch.cuda.synchronize()
        want, want_ids, want_w = big[4].clone(), big[2].clone(), big[3].clone()
        want_small = small[4].clone()
        big[4].fill_(float("nan"))
        big[2].fill_(-1)
        g = _capture(c, stream, lambda: _moe(g4, c, mw, 96, big))
        for rep in range(3):
            big[4].fill_(float("nan"))
            big[2].fill_(-1)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(big[4], want), "replay %d" % rep
            assert torch.equal(big[2], want_ids) and torch.equal(big[3], want_w), "replay %d" % rep
            _moe(g4, c, mw, 4, small)
            torch.cuda.synchronize()
            assert torch.equal(small[4], want_small)
    finally:
        torch.cuda.synchronize()
        c.close()


def test_multi_token_moe_replays(g4, wide_moe_weights):
    """16 tokens at dim 2048 / ff 1408 take the gate+up launch with one wave per
    slot (routing in 512 threads) and the down launch that loops 8-row steps and
    does the weighted sum.  Captured once and replayed three times, with eager
    one-token and grouped calls between the replays: every replay gives the
    eager bits, ids and weights."""
    announce("capture: multi-token MoE replays")
    mw = wide_moe_weights
    c = g4.Context(0)
    stream = torch.cuda.Stream()
    try:
        mid = _io(mw, 16, 7)
        one = _io(mw, 1, 8)
        big = _io(mw, 96, 9)
        _moe(g4, c, mw, 96, big)  # eager: sizes the scratch
        _moe(g4, c, mw, 16, mid)
        _moe(g4, c, mw, 1, one)
        torch.cuda.synchronize()
        want, want_ids, want_w = mid[4].clone(), mid[2].clone(), mid[3].clone()
        want_one, want_big = one[4].clone(), big[4].clone()
        mid[4].fill_(float("nan"))
        mid[2].fill_(-1)
        g = _capture(c, stream, lambda: _moe(g4, c, mw, 16, mid))
        for rep in range(3):
            mid[4].fill_(float("nan"))
            mid[2].fill_(-1)
            mid[3].fill_(0.0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(mid[4], want), "replay %d" % rep
            assert torch.equal(mid[2], want_ids) and torch.equal(mid[3], want_w), "replay %d" % rep
            _moe(g4, c, mw, 1, one)
            _moe(g4, c, mw, 96, big)
            torch.cuda.synchronize()
            assert torch.equal(one[4], want_one) and torch.equal(big[4], want_big)
    finally:
        torch.cuda.synchronize()
        c.close()


def test_growth_under_capture_is_refused_and_reserve_fixes_it(g4, moe_weights):
    announce("capture: growth refused, then reserved")
    mw = moe_weights
    c = g4.Context(0)
    stream = torch.cuda.Stream()
    try:
        io = _io(mw, 8, 3)
        marker = torch.zeros(16, device="cuda")
        assert c.scratch_bytes() == 0

        def refused():
            marker.add_(1.0)  # something for the graph to hold besides the refused call
            with pytest.raises(g4.IllegalArgumentException, match="being captured"):
                _moe(g4, c, mw, 8, io)

        g = _capture(c, stream, refused)
        assert c.scratch_bytes() == 0
        g.replay()
        torch.cuda.synchronize()
        assert float(marker[0]) == 1.0
        # reserve outside the capture, then the same call captures and replays
        c.reserve(8 << 20)
        assert c.scratch_bytes() >= 8 << 20
        _moe(g4, c, mw, 8, io)
        torch.cuda.synchronize()
        want = io[4].clone()
        io[4].fill_(float("nan"))
        g2 = _capture(c, stream, lambda: _moe(g4, c, mw, 8, io))
        for _ in range(3):
            io[4].fill_(float("nan"))
            torch.cuda.synchronize()
            g2.replay()
            torch.cuda.synchronize()
            assert torch.equal(io[4], want)
    finally:
        torch.cuda.synchronize()
        c.close()


def test_host_pointer_calls_are_refused_under_capture(g4, moe_weights):
    announce("capture: host-pointer call refused")
    mw = moe_weights
    c = g4.Context(0)
    stream = torch.cuda.Stream()
    try:
        x = synth.activations(4, "x", mw["dim"])
        y = np.empty(8, np.float32)
        marker = torch.zeros(4, device="cuda")

        def host_matmul():
            # through context c, whose stream is the capturing one
            g4.check(g4.lib().g4_matmul(c.handle, mw["wgu"].handle, 0, x.ctypes.data, y.ctypes.data, 8, mw["dim"]))

        def body():
            marker.add_(1.0)
            with pytest.raises(g4.IllegalArgumentException, match="stream capture"):
                host_matmul()
            with pytest.raises(g4.IllegalArgumentException, match="stream capture"):
                c.sync()

        g = _capture(c, stream, body)
        g.replay()
        torch.cuda.synchronize()
        assert float(marker[0]) == 1.0
        # the context still works eagerly afterwards
        host_matmul()
        assert np.all(np.isfinite(y))
    finally:
        torch.cuda.synchronize()
        c.close()
