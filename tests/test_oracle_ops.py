"""Pins the oracle's restatement of the engine's f32 steps next to the path
(swamp-engine/src/ops.rs:188-220: rmsnorm, silu, mul_in_place,
add_in_place) with closed forms, exact invariances and float64 brute force.
CPU only."""
import numpy as np
import pytest

EPS32 = np.finfo(np.float32).eps


def test_rmsnorm_constant_vector_closed_form(orc):
    # x = c (a power of two), w = 1, eps = 0: mean(x^2) = c^2 exactly, so
    # every output is exactly sign(c); dividing by n - 1 or skipping the
    # square root would not give 1
    for n in (1, 7, 4096):
        for c in (0.25, -8.0, 2.0 ** -20):
            out = orc.rmsnorm(np.full(n, c, np.float32), np.ones(n, np.float32), 0.0)
            assert np.all(out == np.sign(c)), (n, c)


def test_rmsnorm_eps_after_mean(orc):
    # x = 1, eps = 3: ss = 1 + 3 = 4, inv = 0.5 exactly; eps added before the
    # division by n would give a different value for n > 1
    n = 64
    w = np.arange(1, n + 1, dtype=np.float32)
    out = orc.rmsnorm(np.ones(n, np.float32), w, 3.0)
    assert np.array_equal(out, 0.5 * w)


def test_rmsnorm_scale_invariant_when_eps_zero(orc):
    # every step scales by a power of two exactly: rmsnorm(4 x) == rmsnorm(x)
    x = np.random.default_rng(1).standard_normal(4096).astype(np.float32)
    w = np.random.default_rng(2).standard_normal(4096).astype(np.float32)
    a = orc.rmsnorm(x, w, 0.0)
    b = orc.rmsnorm(4.0 * x, w, 0.0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_rmsnorm_vs_f64(orc):
    rng = np.random.default_rng(3)
    for n, eps in ((4096, 1e-5), (8192, 1e-6), (33, 0.5)):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        w = rng.standard_normal(n).astype(np.float32)
        out = orc.rmsnorm(x, w, eps).astype(np.float64)
        x64 = x.astype(np.float64)
        ref = x64 / np.sqrt(np.mean(x64 * x64) + eps) * w
        # sequential f32 sum of squares: relative error <= n eps32, plus the
        # sqrt, division and two products
        assert np.all(np.abs(out - ref) <= (n + 6) * EPS32 * np.abs(ref) + 1e-30)


def test_silu_values(orc):
    v = np.array([0.0, -0.0, 20.0, 100.0, -100.0, -1e4, 1.0, -1.0], np.float32)
    out = orc.silu(v)
    assert out[0] == 0.0 and out[2] == 20.0 and out[3] == 100.0  # exp(-v) below 1 ulp of 1
    assert out[4] <= 0.0 and abs(out[4]) < 1e-40 and out[5] == 0.0
    x = np.linspace(-30, 30, 100001, dtype=np.float32)
    got = orc.silu(x).astype(np.float64)
    x64 = x.astype(np.float64)
    ref = x64 / (1.0 + np.exp(-x64))
    # expf within 1 ulp, then one add and one division rounded
    assert np.all(np.abs(got - ref) <= 4 * EPS32 * np.abs(ref) + 1e-37)


def test_mul_add_in_place_exact(orc):
    rng = np.random.default_rng(4)
    a = rng.standard_normal(10001).astype(np.float32)
    b = rng.standard_normal(10001).astype(np.float32)
    assert np.array_equal(orc.mul_in_place(a, b), a * b)
    assert np.array_equal(orc.add_in_place(a, b), a + b)


@pytest.mark.parametrize("dtype", [2, 12, 14])
def test_fused_compositions_are_linear_in_the_right_places(pkg, orc, dtype):
    """W rmsnorm(x) is invariant to scaling x by a power of two when eps = 0
    (exactly); W (silu(g) * u) is linear in u (2u gives exactly twice)."""
    rows, cols = 24, 1024
    raw = pkg.synth_quantized(dtype, 5, 0.02, rows, cols)
    x = pkg.fill_normal(6, 1.0, 3, cols)
    w = 1.0 + 0.1 * x[2]
    y1 = orc.forward_linear(dtype, raw, orc.rmsnorm(x[0], w, 0.0), rows, cols)
    y2 = orc.forward_linear(dtype, raw, orc.rmsnorm(16 * x[0], w, 0.0), rows, cols)
    assert np.array_equal(y1, y2)
    h1 = orc.mul_in_place(orc.silu(x[0]), x[1])
    h2 = orc.mul_in_place(orc.silu(x[0]), 2 * x[1])
    assert np.array_equal(orc.forward_linear(dtype, raw, h2, rows, cols),
                          2 * orc.forward_linear(dtype, raw, h1, rows, cols))
