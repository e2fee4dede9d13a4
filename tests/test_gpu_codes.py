"""GPU: every weight code decodes exactly.  The kernels turn Q4 nibbles into
fp16 through the fp8 convert (a byte below 16 read as E4M3, scaled by 2^9)
and Q8_0 bytes through an fp16 magic; one-hot activations read the weights
back one column at a time, so each output is a single decoded weight:

  * decode GEMV (fp32 x): y[r] = W[r, j] as the oracle dequantizes it, bit
    for bit for Q4_0 and Q8_0 (d (q - 8) and d q are exact in fp32), within
    4 ulp for Q4_K ((d sc) q - dmin m, whose two products the reference
    rounds separately); equal as numbers, a zero's sign being lost in the
    sum over lanes;
  * small batch (fp16 weights on the matrix cores, 16 one-hot tokens per
    call): y[t, r] = W16[r, j0 + t], the weight rounded once to fp16,
    exactly; W16 is built here from the block fields: fp16(d (q - 8)) for Q4_0,
    fp16(d q) for Q8_0, and for Q4_K fp16(q s - m) with s = fp16(d sc), m =
    fp16(dmin m), the scale pair rounded to fp16 as the kernel forms it;
  * small batch of 2 tokens (the GEMV over both tokens: exact fp16 weight
    pairs 1024 + q times fp16 x scaled by a power of two, the offset taken
    off with the same x): y[t, r] = W[r, j0 + t] as for the decode GEMV,
    Q6_K included (d sc (q - 32) has at most 24 significant bits).

The quantized bytes are random (every code at every byte position), block
scales come from the host quantizer."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
SEED = 0xC0DE


@pytest.fixture(scope="module")
def torch_dev(pkg):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    pkg.init()
    return torch


def random_codes(pkg, dtype, rows, cols, seed):
    """Quantizer scales, random code bytes (Q4_K: random 6-bit scale bytes too)."""
    raw = pkg.synth_quantized(dtype, seed, 0.02, rows, cols).copy()
    rng = np.random.default_rng(seed)
    blk = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210}[dtype]
    first = {Q4_0: 2, Q8_0: 2, Q4_K: 4, Q6_K: 0}[dtype]
    last = blk - 2 if dtype == Q6_K else blk  # Q6_K keeps its d (the last 2 bytes)
    b = raw.reshape(-1, blk)
    b[:, first:last] = rng.integers(0, 256, size=(b.shape[0], last - first), dtype=np.uint8)
    return raw


def f16(u16):
    return np.asarray(u16, dtype=np.uint16).view(np.float16).astype(np.float64)


def w16_expected(orc, dtype, raw, rows, cols):
    """The fp16 weight the small-batch kernel multiplies, per (row, col)."""
    if dtype == Q4_0:
        b = raw.reshape(rows, cols // 32, 18)
        d = f16(b[:, :, 0].astype(np.uint16) | (b[:, :, 1].astype(np.uint16) << 8))
        qs = b[:, :, 2:]
        q = np.empty((rows, cols // 32, 32), dtype=np.float64)
        q[:, :, 0::2] = qs & 15  # interleaved: byte i holds elements 2i, 2i + 1
        q[:, :, 1::2] = qs >> 4
        w = (q - 8.0) * d[:, :, None]
    elif dtype == Q8_0:
        b = raw.reshape(rows, cols // 32, 34)
        d = f16(b[:, :, 0].astype(np.uint16) | (b[:, :, 1].astype(np.uint16) << 8))
        w = b[:, :, 2:].view(np.int8).astype(np.float64) * d[:, :, None]
    else:
        b = raw.reshape(rows, cols // 256, 144)
        d = f16(b[:, :, 0].astype(np.uint16) | (b[:, :, 1].astype(np.uint16) << 8))
        dmin = f16(b[:, :, 2].astype(np.uint16) | (b[:, :, 3].astype(np.uint16) << 8))
        w = np.empty((rows, cols // 256, 256), dtype=np.float64)
        for r in range(rows):
            for s in range(cols // 256):
                sc, mn = orc.unpack_scales_q4k(bytes(b[r, s, 4:16]))
                qs = b[r, s, 16:]
                for g in range(4):  # quarter g: low nibbles sub-block 2g, high 2g + 1
                    by = qs[32 * g:32 * g + 32]
                    for h, q in ((0, by & 15), (1, by >> 4)):
                        j = 2 * g + h
                        s16 = np.float16(d[r, s] * float(sc[j])).astype(np.float64)
                        m16 = np.float16(dmin[r, s] * float(mn[j])).astype(np.float64)
                        w[r, s, 64 * g + 32 * h:64 * g + 32 * h + 32] = q.astype(np.float64) * s16 - m16
    return w.reshape(rows, cols).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
def test_gemv_one_hot_columns(pkg, orc, torch_dev, dtype):
    torch = torch_dev
    rows, cols = 300, 256
    raw = random_codes(pkg, dtype, rows, cols, SEED ^ dtype)
    deq = orc.dequantize(dtype, raw, rows * cols).reshape(rows, cols)
    print(f"[gpu case] gemv one-hot columns dtype {dtype} {rows}x{cols}", flush=True)
    s = torch.cuda.current_stream().cuda_stream
    d_w = torch.from_numpy(raw).cuda()
    d_x = torch.zeros(cols, dtype=torch.float32, device="cuda")
    d_y = torch.empty((cols, rows), dtype=torch.float32, device="cuda")
    for j in range(cols):
        d_x.zero_()
        d_x[j] = 1.0
        pkg.qgemv(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y[j].data_ptr(), rows, cols, s)
    y = d_y.cpu().numpy().T  # y[r, j]
    if dtype == Q4_K:
        tol = 4 * np.spacing(np.maximum(np.abs(deq), np.float32(1e-30)))
        assert np.all(np.abs(y - deq) <= tol), float(np.max(np.abs(y - deq) / tol))
    else:
        # equal as numbers (a zero weight's sign is lost in the lane sum)
        assert np.array_equal(y, deq), float(np.max(np.abs(y - deq)))


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
def test_batched_one_hot_columns(pkg, orc, torch_dev, dtype):
    torch = torch_dev
    rows, cols, n_tok = 300, 1024, 16
    raw = random_codes(pkg, dtype, rows, cols, SEED ^ 0x100 ^ dtype)
    w16 = w16_expected(orc, dtype, raw, rows, cols)
    # the fields decoded here agree with the oracle's dequantization up to
    # the fp16 roundings (Q4_K: also of d sc and dmin m, so relative to the
    # largest weight of each 32-weight group)
    deq = orc.dequantize(dtype, raw, rows * cols).reshape(rows, cols)
    gmax = np.abs(deq).reshape(rows, cols // 32, 32).max(axis=2, keepdims=True)
    err = np.abs(w16 - deq).reshape(rows, cols // 32, 32)
    assert np.all(err <= gmax * 2.0 ** -9 + 2.0 ** -24)
    print(f"[gpu case] batched one-hot columns dtype {dtype} {rows}x{cols}", flush=True)
    s = torch.cuda.current_stream().cuda_stream
    d_w = torch.from_numpy(raw).cuda()
    d_x = torch.zeros((n_tok, cols), dtype=torch.float32, device="cuda")
    got = np.empty((rows, cols), dtype=np.float32)
    d_y = torch.empty((n_tok, rows), dtype=torch.float32, device="cuda")
    for j0 in range(0, cols, n_tok):
        d_x.zero_()
        for t in range(n_tok):
            d_x[t, j0 + t] = 1.0
        pkg.qgemv_batched(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), n_tok,
                          rows, cols, 0, s)
        got[:, j0:j0 + n_tok] = d_y.cpu().numpy().T
    assert np.array_equal(got, w16), float(np.max(np.abs(got - w16)))


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K, Q6_K])
def test_token_gemv_one_hot_columns(pkg, orc, torch_dev, dtype):
    torch = torch_dev
    n_tok = 2
    rows, cols = 300, 512
    raw = random_codes(pkg, dtype, rows, cols, SEED ^ 0x200 ^ dtype)
    deq = orc.dequantize(dtype, raw, rows * cols).reshape(rows, cols)
    print(f"[gpu case] token gemv one-hot columns dtype {dtype} n_tok {n_tok}", flush=True)
    s = torch.cuda.current_stream().cuda_stream
    d_w = torch.from_numpy(raw).cuda()
    d_x = torch.zeros((n_tok, cols), dtype=torch.float32, device="cuda")
    d_y = torch.empty((n_tok, rows), dtype=torch.float32, device="cuda")
    got = np.empty((rows, cols), dtype=np.float32)
    for j0 in range(0, cols, n_tok):
        d_x.zero_()
        nt = min(n_tok, cols - j0)
        for t in range(nt):
            d_x[t, j0 + t] = 1.0
        pkg.qgemv_batched(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), n_tok,
                          rows, cols, 0, s)
        got[:, j0:j0 + nt] = d_y.cpu().numpy().T[:, :nt]
    if dtype == Q4_K:
        tol = 4 * np.spacing(np.maximum(np.abs(deq), np.float32(1e-30)))
        assert np.all(np.abs(got - deq) <= tol), float(np.max(np.abs(got - deq) / tol))
    else:
        assert np.array_equal(got, deq), float(np.max(np.abs(got - deq)))
