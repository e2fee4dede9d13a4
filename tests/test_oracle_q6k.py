"""Pins the oracle's Q6_K restatement (dequant_q6k, swamp-gguf/src/quant/
q6_k.rs:7-56, and the scalar fused GEMV, swamp-kernels/src/fused_gemv_q6k.rs:
248-291) against a block built from the published layout by an independent
packer, the reference's own GEMV test data and test, exact f64 arithmetic
and the reference's private f16 decode.  Also the host Q6_K quantizer
(test-data generator, no reference counterpart).  CPU only."""
import numpy as np
import pytest

Q6_K = 14


def test_q6k_table(orc):
    L = orc.lib()
    assert (L.or_block_size(Q6_K), L.or_type_size(Q6_K)) == (256, 210)
    assert L.or_nbytes_for(Q6_K, 4096 * 128256) == 4096 // 256 * 210 * 128256


def test_q6k_layout_kat(orc, fixtures):
    """Codes (7e + 3) % 64 and signed scales (down to -128) packed by the
    fixture's packer: every output is sc[e // 16] * (q[e] - 32) exactly."""
    k = fixtures["q6_k_layout_kat"]
    raw = np.array(k["raw"], dtype=np.uint8)
    got = orc.dequantize(Q6_K, raw, 256)
    assert got.tolist() == k["expected"]
    # a transposed group, a wrong qh field or an unsigned scale all change
    # some output: the codes are distinct per 16-run and half the scales < 0
    assert len(set(k["q"][:64])) == 64 and min(k["sc"]) == -128


def test_q6k_partial_block_and_short_buffer(orc, fixtures):
    raw = np.array(fixtures["q6_k_layout_kat"]["raw"] * 2, dtype=np.uint8)
    exp = fixtures["q6_k_layout_kat"]["expected"]
    got = orc.dequantize(Q6_K, raw, 300)  # one full block + 44 of the second
    assert got.tolist() == exp + exp[:44]
    with pytest.raises(ValueError):  # BufferTooSmall (q6_k.rs:11-16)
        orc.dequantize(Q6_K, raw[:419], 512)


def test_q6k_values_are_exact(orc, fixtures):
    """(d * sc) * (q - 32) (q6_k.rs:41-44) has at most 11 + 7 + 5 significant
    bits, so every Q6_K weight is the exact product: random blocks (random
    codes, signed scales, normal and subnormal d) decode to the f64 value of
    d * sc[e // 16] * (q[e] - 32), with q read back through the layout."""
    import sys, os
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    from make_fixtures import q6k_codes
    rng = np.random.default_rng(14)
    blocks = rng.integers(0, 256, (64, 210), dtype=np.uint8)
    dcodes = np.concatenate([rng.integers(0x0001, 0x0400, 16),   # subnormal
                             rng.integers(0x0400, 0x7C00, 32),   # normal +
                             rng.integers(0x8400, 0xFC00, 16)])  # normal -
    blocks[:, 208] = dcodes & 0xFF
    blocks[:, 209] = dcodes >> 8
    got = orc.dequantize(Q6_K, blocks.reshape(-1), 64 * 256).reshape(64, 256)
    for b in range(64):
        q, sc, dc = q6k_codes(blocks[b].tolist())
        d = float(np.array([dc], np.uint16).view(np.float16)[0])
        exp = np.array([d * sc[e // 16] * (q[e] - 32) for e in range(256)])
        assert np.array_equal(got[b].astype(np.float64), exp), b


def test_q6k_reference_test_data_values(orc, fixtures):
    """create_test_data (fused_gemv_q6k.rs:329-357) decodes to the values the
    layout gives, row-major."""
    for fx in fixtures["q6_k_reference_test_data"]:
        raw = np.array(fx["raw"], dtype=np.uint8)
        n = fx["n_rows"] * fx["n_blocks"] * 256
        assert orc.dequantize(Q6_K, raw, n).tolist() == fx["w_values"]


def test_q6k_reference_gemv_test(orc, fixtures):
    """test_q6k_bitexact_vs_dequant_scalar (fused_gemv_q6k.rs:358-376):
    fused scalar vs the f32 dot of the dequantized row, |diff| < 1 or
    rel < 1e-4; plus the exact f64 value of the same dot."""
    for fx, fn in zip(fixtures["q6_k_reference_test_data"], (np.sin, np.cos)):
        n_rows, nb = fx["n_rows"], fx["n_blocks"]
        raw = np.array(fx["raw"], dtype=np.uint8)
        x = fn(np.arange(nb * 256, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
        out = orc.fused_gemv_q6k(raw, x, n_rows, nb * 256)
        w = np.array(fx["w_values"], dtype=np.float64).reshape(n_rows, nb * 256)
        for r in range(n_rows):
            dot_ref = np.float32(0)
            for a, b in zip(w[r].astype(np.float32), x):
                dot_ref = np.float32(dot_ref + np.float32(a * b))
            diff = abs(float(out[r]) - float(dot_ref))
            assert diff < 1.0 or diff / max(abs(float(dot_ref)), 1.0) < 1e-4
            exact = float(w[r] @ x.astype(np.float64))
            bound = float(np.abs(w[r]) @ np.abs(x.astype(np.float64)))
            assert abs(float(out[r]) - exact) <= nb * 256 * 2 * np.finfo(np.float32).eps * bound


def test_q6k_private_f16_decode(orc):
    """f16_to_f32_raw (fused_gemv_q6k.rs:11-21) agrees with the exact decode
    on every code with exponent field 1..30, which is why the oracle can use
    the exact decode; zero and subnormal codes decode to about -2^114."""
    codes = np.arange(65536, dtype=np.uint16)
    exp = (codes >> 10) & 0x1F
    exact = codes.view(np.float16).astype(np.float32)
    raw = np.array([orc.q6k_f16_raw(int(c)) for c in codes], dtype=np.float32)
    normal = (exp >= 1) & (exp <= 30)
    assert np.array_equal(raw[normal].view(np.uint32), exact[normal].view(np.uint32))
    assert orc.q6k_f16_raw(0x0000) == -(2.0 ** 114)
    assert orc.q6k_f16_raw(0x7C00) == 65536.0  # inf decodes as a finite value


def _q6k(pkg, rows, cols, seed, sigma=0.02):
    return pkg.synth_quantized(Q6_K, seed, sigma, rows, cols)


@pytest.mark.parametrize("cols", [256, 512, 1280])
def test_q6k_forward_linear_vs_f64(pkg, orc, cols):
    rows = 29
    raw = _q6k(pkg, rows, cols, 40 + cols)
    x = pkg.fill_normal(41, 1.0, 1, cols)[0]
    y = orc.forward_linear(Q6_K, raw, x, rows, cols, 3)
    deq = orc.dequantize(Q6_K, raw, rows * cols).reshape(rows, cols).astype(np.float64)
    y64 = deq @ x.astype(np.float64)
    bound = np.abs(deq) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(y - y64) <= cols * np.finfo(np.float32).eps * bound + 1e-12)


def test_q6k_forward_linear_is_fused_scalar_and_partition_free(pkg, orc):
    rows, cols = 37, 1024
    raw = _q6k(pkg, rows, cols, 7)
    x = pkg.fill_normal(8, 1.0, 1, cols)[0]
    f = orc.fused_gemv_q6k(raw, x, rows, cols)
    for nt in (1, 2, 5, 16):
        y = orc.forward_linear(Q6_K, raw, x, rows, cols, nt)
        assert np.array_equal(y.view(np.uint32), f.view(np.uint32))


def test_q6k_batch_is_per_token(pkg, orc):
    """fallback_gemv's Q6_K arm (linear.rs:336-364): fused_gemv_q6k per token,
    written over the output."""
    rows, cols, bs = 16, 512, 4
    raw = _q6k(pkg, rows, cols, 9)
    xs = pkg.fill_normal(10, 1.0, bs, cols)
    outs = orc.forward_linear_batch(Q6_K, raw, xs, rows, cols, 2)
    for t in range(bs):
        single = orc.fused_gemv_q6k(raw, xs[t], rows, cols)
        assert np.array_equal(outs[t].view(np.uint32), single.view(np.uint32))


def test_q6k_shape_errors(pkg, orc):
    raw = _q6k(pkg, 4, 256, 1)
    with pytest.raises(ValueError):
        orc.fused_gemv_q6k(raw, np.zeros(300, np.float32), 4, 300)  # n_cols % 256
    with pytest.raises(ValueError):
        orc.forward_linear(Q6_K, raw, np.zeros(128, np.float32), 4, 256)  # bail!


def test_q6k_quantizer_round_trip(pkg, orc):
    """The host quantizer (test data only): every weight within one step of
    its source, the step being |d * sc| of its 16-run; scales of both signs
    and subnormal d occur at sigma 0.02."""
    rows, cols = 8, 2048
    src = pkg.fill_normal(77, 0.02, rows, cols)
    raw = pkg.quantize(Q6_K, src)
    assert np.array_equal(raw, _q6k(pkg, rows, cols, 77))  # synth = fill + quantize
    deq = orc.dequantize(Q6_K, raw, rows * cols).reshape(rows, cols)
    blocks = raw.reshape(-1, 210)
    sc = blocks[:, 192:208].view(np.int8).astype(np.float64)
    d = blocks[:, 208:210].copy().view(np.float16).astype(np.float64)[:, 0]
    step = np.repeat(np.abs(d[:, None] * sc), 16, axis=1).reshape(rows, cols)
    assert np.all(np.abs(deq - src) <= step * 1.0001)
    assert np.abs(deq - src).mean() < 0.3 * step.mean()
    assert (sc < 0).any() and (sc > 0).any()
    assert (np.abs(d) < 2.0 ** -14).any()  # subnormal f16 d


def test_q6k_quantizer_zero_block(pkg, orc):
    raw = pkg.quantize(Q6_K, np.zeros((1, 256), np.float32))
    assert not raw.any()
    assert not orc.dequantize(Q6_K, raw, 256).any()
