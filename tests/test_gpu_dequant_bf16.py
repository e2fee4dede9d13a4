"""GPU checks of the bf16 dequantization (`swamp_qdequant_bf16`), the pass the
prefill GEMM's dequantize-once route runs before its bf16 library GEMM.

  * Bit-exact: every output is the oracle's dequantized fp32 value
    (quant::dequantize, swamp-gguf/src/quant/mod.rs:18-33) rounded to
    nearest even, computed here in numpy from the fp32 bits; NaN positions
    identical.  Synthetic weights, ragged block counts (the last workgroup
    partly empty) and uniformly random block bytes (every f16 scale code).
  * Both prefill GEMM routes multiply exactly these bf16 weights: the fused
    kernel (512 tokens) and the dequantize-once route (2048 tokens; Q6_K at
    any size) agree with a float64 product of the bf16 weights and the bf16
    x within 1e-5 of ||W_r|| ||x|| (fp32 accumulation order only), far
    tighter than the 1e-3 contract: weights rounded another way (truncated,
    or from fp32 values with a wrong scale) would miss it by two orders of
    magnitude.  Single values are pinned bit for bit by the tests above."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 2, 8, 12, 14, 30
SEED = 0xBF16
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}


@pytest.fixture(scope="module")
def torch_dev(pkg):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    pkg.init()
    return torch


def stream(torch):
    return torch.cuda.current_stream().cuda_stream


def say(*a):
    print("[gpu case]", *a, flush=True)


def rne_bf16(f32):
    """fp32 -> bf16 bits, round to nearest even (finite values; NaN handled
    by the caller)."""
    b = np.ascontiguousarray(f32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def device_bf16(pkg, torch, dtype, raw, n, offset=0):
    """swamp_qdequant_bf16 on raw placed `offset` bytes into its device
    buffer; returns the uint16 bits."""
    buf = np.zeros(raw.size + offset, dtype=np.uint8)
    buf[offset:] = raw
    d_raw = torch.from_numpy(buf).cuda()
    d_out = torch.empty(n, dtype=torch.int16, device="cuda")
    pkg.qdequant_bf16(dtype, d_raw.data_ptr() + offset, raw.size, d_out.data_ptr(), n,
                      stream(torch))
    torch.cuda.synchronize()
    return d_out.cpu().numpy().view(np.uint16)


def check_bits(got, ref_f32):
    nan = np.isnan(ref_f32)
    got_nan = ((got & 0x7F80) == 0x7F80) & ((got & 0x007F) != 0)
    assert np.array_equal(got_nan, nan)
    assert np.array_equal(got[~nan], rne_bf16(ref_f32[~nan]))


@pytest.mark.parametrize("dtype,n_blocks", [(Q4_0, 1), (Q4_0, 257), (Q4_0, 4096 * 128),
                                            (Q8_0, 1), (Q8_0, 1000), (Q8_0, 4096 * 32),
                                            (Q4_K, 1), (Q4_K, 33), (Q4_K, 16 * 1024),
                                            (Q6_K, 1), (Q6_K, 1001), (Q6_K, 16 * 1024)])
def test_dequant_bf16_bit_exact(pkg, orc, torch_dev, dtype, n_blocks):
    bs, _ = BLOCK[dtype]
    n = n_blocks * bs
    raw = pkg.synth_quantized(dtype, SEED ^ n_blocks, 0.02, 1, n)
    say("dequant bf16", dtype, n)
    check_bits(device_bf16(pkg, torch_dev, dtype, raw, n), orc.dequantize(dtype, raw, n))


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K, Q6_K])
def test_dequant_bf16_random_bytes(pkg, orc, torch_dev, dtype):
    """Uniformly random block bytes: subnormal, infinite and NaN f16 scales,
    every 6-bit code, signed Q6_K scales.  Q6_K is read from a base 2 bytes
    past a 4-byte boundary (its blocks are only 2-byte aligned)."""
    bs, ts = BLOCK[dtype]
    nblk = 20000
    raw = np.random.default_rng(dtype ^ 0xB).integers(0, 256, nblk * ts, dtype=np.uint8)
    n = nblk * bs
    say("dequant bf16 random bytes", dtype)
    got = device_bf16(pkg, torch_dev, dtype, raw, n, offset=2 if dtype == Q6_K else 0)
    check_bits(got, orc.dequantize(dtype, raw, n))


@pytest.mark.parametrize("dtype,m,rows,cols", [(Q4_0, 512, 1024, 1024), (Q4_0, 2048, 1024, 1024),
                                               (Q8_0, 512, 1280, 1024), (Q8_0, 2048, 1280, 1024),
                                               (Q4_K, 512, 1024, 2048), (Q4_K, 2048, 1024, 2048),
                                               (Q6_K, 64, 1024, 1024)])
def test_gemm_routes_use_the_bf16_weights(pkg, orc, torch_dev, errlog, dtype, m, rows, cols):
    torch = torch_dev
    raw = pkg.synth_quantized(dtype, SEED ^ (m << 20) ^ rows, 0.02, rows, cols)
    x = pkg.fill_normal(SEED ^ m, 1.0, m, cols)
    xb = pkg.to_bf16_bits(x)
    x_fed = bf16_to_f32(xb)
    say("gemm routes bf16 weights", dtype, m, rows, cols)
    d_w = torch.from_numpy(raw).cuda()
    d_x = torch.from_numpy(xb.view(np.int16)).cuda()
    d_y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
    pkg.qgemm(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), BF16, d_y.data_ptr(), m, rows, cols,
              stream(torch))
    torch.cuda.synchronize()
    y = d_y.cpu().numpy()
    w16 = bf16_to_f32(rne_bf16(orc.dequantize(dtype, raw, rows * cols))).reshape(rows, cols)
    toks = sorted({0, 1, m // 3, m - 1})
    ref = x_fed[toks].astype(np.float64) @ w16.T.astype(np.float64)
    err = errlog(f"gemm bf16-weight product {dtype} {m}x{rows}x{cols}",
                 orc.normalized_error(y[toks], ref, w16, x_fed[toks]), path="gemm_bf16_exact")
    assert err <= 1e-5
