"""Pins the CPU oracle (a C restatement of the reference's scalar path)
against the reference's own test fixtures, known answers, library routines
and closed forms.  CPU only."""
import numpy as np
import pytest

Q4_0, Q8_0, Q4_K = 2, 8, 12


# ---------------------------------------------------------------- A1 table

def test_dtype_table(orc):
    L = orc.lib()
    # GGUF block geometry of the three path dtypes (swamp-gguf/src/dtype.rs)
    assert (L.or_block_size(Q4_0), L.or_type_size(Q4_0)) == (32, 18)
    assert (L.or_block_size(Q8_0), L.or_type_size(Q8_0)) == (32, 34)
    assert (L.or_block_size(Q4_K), L.or_type_size(Q4_K)) == (256, 144)
    assert L.or_nbytes_for(Q4_0, 4096 * 4096) == 9_437_184
    assert L.or_nbytes_for(Q4_0, 33) == 36  # ceil(n / bs) * ts
    assert L.or_block_size(99) == 0


# ------------------------------------------------------------ A2 f16 decode

def test_f16_exhaustive_vs_numpy(orc):
    codes = np.arange(65536, dtype=np.uint16)
    got = orc.f16_to_f32(codes)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_exhaustive_vs_f16c(orc):
    codes = np.arange(65536, dtype=np.uint16)
    hw = orc.f16_to_f32_hw(codes)
    if hw is None:
        pytest.skip("host CPU has no F16C")
    got = orc.f16_to_f32(codes)
    # bit-identical including NaN payloads (quiet bit set)
    assert np.array_equal(got.view(np.uint32), hw.view(np.uint32))


# --------------------------------------------------------- A3-A5 dequantize

def test_q4_0_interleave_kat(orc, fixtures):
    k = fixtures["q4_0_kat"]
    raw = np.array(k["raw"], dtype=np.uint8)
    got = orc.dequantize(Q4_0, raw, 64)
    assert got.tolist() == k["expected"]


def test_q4_0_partial_block_and_short_buffer(orc, fixtures):
    raw = np.array(fixtures["q4_0_kat"]["raw"], dtype=np.uint8)
    got = orc.dequantize(Q4_0, raw, 40)  # 1 full block + 8 of the second
    assert got.tolist() == fixtures["q4_0_kat"]["expected"][:40]
    with pytest.raises(ValueError):  # BufferTooSmall (q4_0.rs:15-20)
        orc.dequantize(Q4_0, raw[:35], 64)


def test_q8_0_kat(orc, fixtures):
    k = fixtures["q8_0_kat"]
    got = orc.dequantize(Q8_0, np.array(k["raw"], dtype=np.uint8), 64)
    assert got.tolist() == k["expected"]


def test_q4_k_layout_kat(orc, fixtures):
    k = fixtures["q4_k_layout_kat"]
    got = orc.dequantize(Q4_K, np.array(k["raw"], dtype=np.uint8), 256)
    assert got.tolist() == k["expected"]


def test_q4_k_scales_from_reference_packer(orc, fixtures):
    k = fixtures["q4_k_scale_kat"]
    raw = np.array(k["raw"], dtype=np.uint8)
    s, m = orc.unpack_scales_q4k(raw[4:16].tobytes())
    assert s.tolist() == k["scales"] and m.tolist() == k["mins"]
    got = orc.dequantize(Q4_K, raw, 256)
    assert np.allclose(got, k["expected"], rtol=0, atol=0)  # exact: small binary values


def test_q4_k_unpack_random_roundtrip(orc):
    # pack random 6-bit codes with the reference's packer layout, unpack
    rng = np.random.default_rng(3)
    for _ in range(200):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        b = [0] * 12
        for j in range(4):
            b[j] = int((sc[j] & 0x3F) | ((sc[4 + j] >> 4) << 6))
            b[4 + j] = int((mn[j] & 0x3F) | ((mn[4 + j] >> 4) << 6))
            b[8 + j] = int((sc[4 + j] & 0xF) | ((mn[4 + j] & 0xF) << 4))
        s, m = orc.unpack_scales_q4k(bytes(b))
        assert s.tolist() == sc.tolist() and m.tolist() == mn.tolist()


def test_q4_k_two_roundings(orc):
    # w = (d*sc)*q - dmin*m with separate roundings: pick values where a
    # fused multiply-subtract would differ in the last bit.
    d = np.float32(0.1).astype(np.float16)
    dmin = np.float32(0.3).astype(np.float16)
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = np.frombuffer(d.tobytes(), dtype=np.uint8)
    blk[2:4] = np.frombuffer(dmin.tobytes(), dtype=np.uint8)
    blk[4:8] = 37
    blk[8:12] = 11
    blk[16:] = np.arange(128, dtype=np.uint8)
    got = orc.dequantize(Q4_K, blk, 256)
    sv = np.float32(d) * np.float32(37)
    mv = np.float32(dmin) * np.float32(11)
    q = (np.arange(128) & 15).astype(np.float32)
    exp = (sv * q).astype(np.float32) - mv  # numpy float32: two roundings
    assert np.array_equal(got[:32].view(np.uint32), exp[:32].view(np.uint32))


# -------------------------------------------------------------- A7 GEMV

def test_reference_gemv_fixtures_closed_form(orc, fixtures):
    for fx in fixtures["gemv_fixtures"]:
        w = np.array(fx["w"], dtype=np.uint8)
        x = np.array(fx["x"], dtype=np.float32)
        n = fx["n_rows"]
        y = orc.fused_gemv_q4k(w, x, n, 256)
        # every dequantized weight equals the closed-form value exactly
        deq = orc.dequantize(Q4_K, w, n * 256).reshape(n, 256)
        for r in range(n):
            assert np.all(deq[r] == np.float32(fx["w_value"][r])) or np.allclose(
                deq[r], fx["w_value"][r], rtol=1e-6)
        bound = np.abs(np.array(fx["w_value"]))[:, None] * np.abs(x)[None, :]
        tol = 256 * 2 * np.finfo(np.float32).eps * bound.sum(axis=1)
        assert np.all(np.abs(y - np.array(fx["y"])) <= tol + 1e-6)


def test_reference_batched_vs_single(orc, fixtures):
    # fused_gemv_q4k.rs:742-790: batch-1 batched == single within 0.01
    for fx in fixtures["gemv_fixtures"]:
        w = np.array(fx["w"], dtype=np.uint8)
        x = np.array(fx["x"], dtype=np.float32)[None, :].copy()
        n = fx["n_rows"]
        single = orc.fused_gemv_q4k(w, x[0], n, 256)
        outs = np.zeros((1, n), dtype=np.float32)
        orc.fused_gemv_q4k_batched(w, x, outs, n, 256)
        assert np.all(np.abs(outs[0] - single) < 0.01)


def _rand_q(pkg, dtype, rows, cols, seed):
    return pkg.synth_quantized(dtype, seed, 0.02, rows, cols)


@pytest.mark.parametrize("dtype,cols", [(Q4_0, 96), (Q4_0, 512), (Q8_0, 64), (Q8_0, 320),
                                        (Q4_K, 256), (Q4_K, 768)])
def test_forward_linear_vs_f64(pkg, orc, dtype, cols):
    rows = 37
    raw = _rand_q(pkg, dtype, rows, cols, 11 + cols)
    x = pkg.fill_normal(99, 1.0, 1, cols)[0]
    y = orc.forward_linear(dtype, raw, x, rows, cols, 3)
    deq = orc.dequantize(dtype, raw, rows * cols).reshape(rows, cols).astype(np.float64)
    y64 = deq @ x.astype(np.float64)
    bound = np.abs(deq) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(y - y64) <= cols * np.finfo(np.float32).eps * bound + 1e-12)


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
def test_forward_linear_partition_independent(pkg, orc, dtype):
    rows, cols = 101, 512
    raw = _rand_q(pkg, dtype, rows, cols, 5)
    x = pkg.fill_normal(6, 1.0, 1, cols)[0]
    ys = [orc.forward_linear(dtype, raw, x, rows, cols, nt) for nt in (1, 2, 6, 16)]
    for y in ys[1:]:
        assert np.array_equal(y.view(np.uint32), ys[0].view(np.uint32))


def test_forward_linear_q4k_is_fused_scalar(pkg, orc):
    rows, cols = 20, 1024
    raw = _rand_q(pkg, Q4_K, rows, cols, 8)
    x = pkg.fill_normal(9, 1.0, 1, cols)[0]
    a = orc.forward_linear(Q4_K, raw, x, rows, cols, 4)
    b = orc.fused_gemv_q4k(raw, x, rows, cols)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_multi_equals_concatenated_single(pkg, orc):
    cols = 512
    mats = [_rand_q(pkg, Q4_K, r, cols, 20 + r) for r in (3, 8, 5)]
    x = pkg.fill_normal(1, 1.0, 1, cols)[0]
    outs = orc.fused_gemv_q4k_multi(mats, x, [3, 8, 5], cols)
    for w, r, o in zip(mats, (3, 8, 5), outs):
        s = orc.fused_gemv_q4k(w, x, r, cols)
        assert np.array_equal(o.view(np.uint32), s.view(np.uint32))


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
def test_batch_linearity_and_tokens(pkg, orc, dtype):
    rows, cols, bs = 24, 512, 5
    raw = _rand_q(pkg, dtype, rows, cols, 31)
    xs = pkg.fill_normal(32, 1.0, bs, cols)
    outs = orc.forward_linear_batch(dtype, raw, xs, rows, cols, 2)
    for t in range(bs):
        single = orc.forward_linear(dtype, raw, xs[t], rows, cols, 1)
        assert np.allclose(outs[t], single, rtol=1e-5, atol=1e-6)
    # linearity: W(a x) = a W x for a power of two (exact)
    y2 = orc.forward_linear(dtype, raw, 2.0 * xs[0], rows, cols, 1)
    y1 = orc.forward_linear(dtype, raw, xs[0], rows, cols, 1)
    assert np.array_equal(y2, 2.0 * y1)


def test_shape_errors(pkg, orc):
    raw = _rand_q(pkg, Q4_K, 4, 256, 1)
    x = np.zeros(255, dtype=np.float32)
    with pytest.raises(ValueError):
        orc.fused_gemv_q4k(raw, x, 4, 255)  # n_cols % 256 != 0
    with pytest.raises(ValueError):  # x shorter than n_cols: bail!
        orc.forward_linear(Q4_K, raw, np.zeros(128, np.float32), 4, 256)


# ------------------------------------------------------------ A17 int8 dot

def test_int8_dot_reference_kat(orc, fixtures):
    s = 0xDEAD_BEEF_1234_5678
    for t in fixtures["int8_dot_kat"]:
        w, s = orc.xorshift64_i8(s, t["k"])
        a, s = orc.xorshift64_i8(s, t["k"])
        assert w.tolist() == t["w"] and a.tolist() == t["a"]
        exact = int(np.dot(w.astype(np.int64), a.astype(np.int64)))
        assert exact == t["dot"]
        assert orc.gemv_q8_dot(w, a, 1.0) == float(np.float32(t["dot"]))
    assert orc.gemv_q8_dot(np.zeros(0, np.int8), np.zeros(0, np.int8), 1.0) == 0.0
