"""The committed golden fixtures (tests/golden/fixtures.npz) through the GPU path.

Every format's small cases (512 and 1408 columns on the fast kernels, 288
columns on the per-element path) must land within 1e-5 * sum|w_i x_i| of the
committed fp64 dots, and the routed MoE case within its committed bound, with
the routing (ids and gate weights) equal to the committed one."""
import numpy as np
import pytest

from conftest import announce
from test_golden import dot_cases, load_fixtures

pytestmark = pytest.mark.gpu


def test_fixture_dots(g4, ctx):
    fx = load_fixtures()
    for key, t, rows, cols in dot_cases(fx):
        announce("golden fixture %s" % key)
        w = g4.FloatTensorFactory.create(ctx, t, fx[key + ".raw"], rows * cols)
        y = np.empty(rows, np.float32)
        w.matmul(fx[key + ".x"], y, rows, cols)
        err = np.abs(y.astype(np.float64) - fx[key + ".y64"])
        assert np.all(err <= 1e-5 * fx[key + ".ab"]), key
        w.free()


def test_fixture_moe(g4, ctx):
    announce("golden fixture moe")
    fx = load_fixtures()
    E, dim, ff, T, k = (int(v) for v in fx["moe.shape"])
    wgu = g4.FloatTensorFactory.create(ctx, 12, fx["moe.gate_up"], E * 2 * ff * dim)
    wdn = g4.FloatTensorFactory.create(ctx, 12, fx["moe.down"], E * dim * ff)
    Y, ids, w = g4.moe_routed(ctx, wgu, wdn, fx["moe.x"], fx["moe.logits"], k, True, dim, ff)
    assert np.array_equal(ids, fx["moe.ids"])
    assert np.array_equal(w.view(np.uint32), fx["moe.w"].view(np.uint32))
    assert np.all(np.abs(Y.astype(np.float64) - fx["moe.y64"]) <= 1e-5 * fx["moe.bound"])
    wgu.free()
    wdn.free()
