"""Host quantizers and synthetic data of libswamp_quant.so (the reference has
no quantizer: these are pinned by IEEE library routines, round-trip bounds
and determinism, not by reference parity -- "parity unpinned")."""
import hashlib
import json
import os

import numpy as np
import pytest

Q4_0, Q8_0, Q4_K = 2, 8, 12
HERE = os.path.dirname(os.path.abspath(__file__))


def test_f32_to_f16_matches_numpy(pkg):
    L = pkg.quant_lib()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504, 65520, 65519.99, 1e-8, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                  np.inf, -np.inf, 6.1e-5, 6.0e-5], dtype=np.float32)]).astype(np.float32)
    got = np.array([L.swamp_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    with np.errstate(over='ignore'):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_bf16_rne(pkg):
    vals = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.0e38, 1e-40, 0.0, 1.0 + 2 ** -8,
                     1.0 + 3 * 2 ** -9], dtype=np.float32)
    got = pkg.to_bf16_bits(vals)
    # RNE by hand on the bit patterns
    u = vals.view(np.uint32).astype(np.uint64)
    exp = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(got, exp)


def test_fill_normal_stats_and_determinism(pkg):
    a = pkg.fill_normal(1234, 0.02, 64, 4096, n_threads=1)
    b = pkg.fill_normal(1234, 0.02, 64, 4096, n_threads=7)
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 1e-3 and abs(a.std() - 0.02) < 2e-4


# rounding error (half a step; a full step on the clipped +8 side of Q4_0),
# plus |q| * (f16(d) - d) <= |q|max * 2^-11 * d
@pytest.mark.parametrize("dtype,bound", [(Q4_0, 1.0 + 8 / 2048), (Q8_0, 0.5 + 127 / 2048)])
def test_roundtrip_bound_q4_0_q8_0(pkg, orc, dtype, bound):
    rows, cols = 64, 1024
    w = pkg.fill_normal(7, 0.02, rows, cols)
    raw = pkg.quantize(dtype, w)
    deq = orc.dequantize(dtype, raw, rows * cols).reshape(rows, cols)
    blocks = w.reshape(rows, -1, 32)
    amax = np.abs(blocks).max(axis=2, keepdims=True)
    step = amax / (8.0 if dtype == Q4_0 else 127.0)
    err = np.abs(deq.reshape(rows, -1, 32) - blocks)
    # |x - deq(q(x))| <= bound * step (+ f16 rounding of d)
    assert np.all(err <= bound * step * (1 + 2e-3) + 1e-9)


def test_roundtrip_bound_q4_k(pkg, orc):
    rows, cols = 32, 2048
    w = pkg.fill_normal(8, 0.02, rows, cols)
    raw = pkg.quantize(Q4_K, w)
    deq = orc.dequantize(Q4_K, raw, rows * cols).reshape(rows, cols)
    sub = w.reshape(rows, -1, 32)
    rng_ = sub.max(axis=2, keepdims=True) - np.minimum(sub.min(axis=2, keepdims=True), 0)
    err = np.abs(deq.reshape(rows, -1, 32) - sub)
    # one quantization step of the sub-block (range / 15, codes rounded up)
    assert np.all(err <= rng_ / 15 * 1.6 + 1e-6)
    rel = np.linalg.norm(deq - w) / np.linalg.norm(w)
    assert rel < 0.12


def test_synth_equals_fill_then_quantize(pkg):
    for dt in (Q4_0, Q8_0, Q4_K, 14):
        a = pkg.synth_quantized(dt, 77, 0.02, 16, 512, n_threads=3)
        b = pkg.quantize(dt, pkg.fill_normal(77, 0.02, 16, 512))
        assert np.array_equal(a, b)


def test_quantize_rejects_bad_shapes(pkg):
    L = pkg.quant_lib()
    src = np.zeros((2, 48), dtype=np.float32)
    dst = np.zeros(1024, dtype=np.uint8)
    assert L.swamp_quantize(Q4_0, src.ctypes.data, dst.ctypes.data, 2, 48, 1) == -1
    assert L.swamp_quantize(13, src.ctypes.data, dst.ctypes.data, 2, 64, 1) == -2  # Q5_K
    assert L.swamp_quantize(14, src.ctypes.data, dst.ctypes.data, 2, 64, 1) == -1  # Q6_K: cols % 256


def test_generator_fixture_hashes(pkg):
    """Pins the synthetic-weight generator: sha256 of the first 4 KiB of
    each benchmark matrix's bytes (tests/golden/generator_hashes.json)."""
    with open(os.path.join(HERE, "golden", "generator_hashes.json")) as f:
        ref = json.load(f)
    for e in ref["entries"]:
        raw = pkg.synth_quantized(e["dtype"], int(e["seed"]), e["sigma"], e["rows"], e["cols"])
        assert hashlib.sha256(raw[:4096].tobytes()).hexdigest() == e["sha256"], e
