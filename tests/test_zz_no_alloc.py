"""g4_moe_routed_dev_noalloc: the routed MoE block with its intermediates in the
library's fixed per-GPU scratch instead of the context's (no device allocation).

It must return the same bits as g4_moe_routed_dev (the same kernels), also on a
second call with fewer tokens (the fixed scratch keeps the previous call's
contents, which must not leak into the result), and refuse a call whose
intermediates exceed the fixed size.  Called through the C ABI."""
import numpy as np
import pytest
import torch

import synth
from conftest import announce

pytestmark = pytest.mark.gpu

Q4_K = 12


@pytest.fixture(scope="module")
def experts(g4, ctx):
    E, dim, ff = 32, 2048, 1408
    gu = synth.q4_k(57, "gu", E * 2 * ff * dim)
    dn = synth.q4_k(57, "dn", E * dim * ff)
    wgu = g4.FloatTensorFactory.create(ctx, Q4_K, gu, E * 2 * ff * dim)
    wdn = g4.FloatTensorFactory.create(ctx, Q4_K, dn, E * dim * ff)
    yield dict(E=E, dim=dim, ff=ff, k=8, wgu=wgu, wdn=wdn)
    wgu.free()
    wdn.free()


def _call(g4, name, ctx, ex, T, X, lg, scale, ids, w, Y):
    fn = getattr(g4.lib(), name)
    return fn(ctx.handle, ex["wgu"].handle, ex["wdn"].handle, X.data_ptr(), T, ex["dim"], ex["ff"], lg.data_ptr(),
              ex["E"], ex["k"], 1, scale.data_ptr() if scale is not None else None, ids.data_ptr(), w.data_ptr(),
              Y.data_ptr())


def _bufs(ex, T, seed):
    X = torch.from_numpy(synth.activations(seed, "x", T * ex["dim"]).reshape(T, ex["dim"])).cuda()
    lg = torch.from_numpy(synth.activations(seed, "lg", T * ex["E"]).reshape(T, ex["E"])).cuda()
    outs = []
    for _ in range(2):
        outs.append((torch.full((T, ex["k"]), -7, dtype=torch.int32, device="cuda"),
                     torch.full((T, ex["k"]), float("nan"), dtype=torch.float32, device="cuda"),
                     torch.full((T, ex["dim"]), float("nan"), dtype=torch.float32, device="cuda")))
    return X, lg, outs


@pytest.mark.parametrize("with_scale", [False, True])
def test_noalloc_matches_the_allocating_entry_point(g4, ctx, experts, with_scale):
    ex = experts
    scale = (torch.from_numpy(np.abs(synth.activations(58, "sc", ex["E"])) + 0.5).cuda() if with_scale else None)
    # each call smaller than the one before; 48 tokens run the experts grouped
    # (k_route, the 16-pair tiles, k_gelu_mul) with their intermediates in the
    # fixed scratch
    for T, seed in ((48, 5), (16, 1), (3, 2)):
        announce("noalloc moe T=%d scale=%s" % (T, with_scale))
        X, lg, ((i0, w0, y0), (i1, w1, y1)) = _bufs(ex, T, seed + (10 if with_scale else 0))
        assert _call(g4, "g4_moe_routed_dev", ctx, ex, T, X, lg, scale, i0, w0, y0) == 0, g4.last_error()
        assert _call(g4, "g4_moe_routed_dev_noalloc", ctx, ex, T, X, lg, scale, i1, w1, y1) == 0, g4.last_error()
        torch.cuda.synchronize()
        assert torch.equal(i0, i1)
        assert torch.equal(w0.view(torch.int32), w1.view(torch.int32))
        assert torch.equal(y0.view(torch.int32), y1.view(torch.int32))
        assert bool(torch.isfinite(y1).all())


def test_noalloc_refuses_intermediates_past_its_fixed_size(g4, ctx, experts):
    announce("noalloc moe oversize")
    ex = experts
    # 4 * T * k * (3 * ff + dim) bytes: 100 tokens x 8 slots need about 20 MB > 16 MiB
    T = 100
    X, lg, ((ids, w, Y), _) = _bufs(ex, T, 3)
    Y.zero_()
    torch.cuda.synchronize()
    rc = _call(g4, "g4_moe_routed_dev_noalloc", ctx, ex, T, X, lg, None, ids, w, Y)
    assert rc == -1 and "allocation-free" in g4.last_error()
    torch.cuda.synchronize()
    assert bool((Y == 0).all())  # nothing was launched
    # the Python wrapper maps it to the reference's IllegalArgumentException
    with pytest.raises(g4.IllegalArgumentException):
        g4.moe_routed_dev_noalloc(ctx, ex["wgu"], ex["wdn"], X, T, ex["dim"], ex["ff"], lg, ex["E"], ex["k"], True,
                                  ids, w, Y)
    # and the entry point still works at a size that fits
    T = 4
    X, lg, ((i0, w0, y0), (i1, w1, y1)) = _bufs(ex, T, 4)
    g4.moe_routed_dev(ctx, ex["wgu"], ex["wdn"], X, T, ex["dim"], ex["ff"], lg, ex["E"], ex["k"], True, i0, w0, y0)
    g4.moe_routed_dev_noalloc(ctx, ex["wgu"], ex["wdn"], X, T, ex["dim"], ex["ff"], lg, ex["E"], ex["k"], True,
                              i1, w1, y1)
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int32), y1.view(torch.int32))
