"""The CPU baseline's build of the oracle (gcc -O3 -march=native
-ffp-contract=off, made on the host that runs bench.py) computes exactly
what the portable checker build computes: no contraction and no fast-math,
so optimisation may change speed but not one bit of the results."""
import importlib.util
import os

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_native_build_is_bit_identical(pkg, orc):
    spec = importlib.util.spec_from_file_location("swamp_oracle_native_check",
                                                  os.path.join(REPO, "oracle", "oracle.py"))
    nat = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(nat)
    desc = nat.use_native_build()
    assert "-march=native" in desc and "-ffp-contract=off" in desc, desc
    for dt, rows, cols in [(pkg.Q4_0, 333, 4096), (pkg.Q8_0, 200, 2048), (pkg.Q4_K, 257, 2048)]:
        raw = pkg.synth_quantized(dt, 0xBA5E ^ dt, 0.02, rows, cols)
        xs = pkg.fill_normal(0xBA5E, 1.0, 3, cols)
        for nt in (1, 6):
            a = orc.forward_linear(dt, raw, xs[0], rows, cols, nt)
            b = nat.forward_linear(dt, raw, xs[0], rows, cols, nt)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (dt, nt)
            a = orc.forward_linear_batch(dt, raw, xs, rows, cols, nt)
            b = nat.forward_linear_batch(dt, raw, xs, rows, cols, nt)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (dt, nt)
        assert np.array_equal(orc.dequantize(dt, raw, rows * cols).view(np.uint32),
                              nat.dequantize(dt, raw, rows * cols).view(np.uint32))
