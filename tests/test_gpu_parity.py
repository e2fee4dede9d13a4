"""GPU parity: every entry point of libswamp_gpu.so against the CPU oracle on
identical seeded inputs.  Gates (from the path's contract):
  * dequantization is bit-identical (NaN positions identical);
  * matmul outputs satisfy max_r |y - y_ref| / (||W_r|| ||x||) <= 1e-3, with
    W the oracle-dequantized weights and x the activations actually fed
    (bf16-rounded for the prefill GEMM).
Large shapes run on the GPU in full; the oracle checks row/token subsets
and the size-independent properties (linearity, batch = per-token)."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K, F32, F16, BF16 = 2, 8, 12, 14, 0, 1, 30
TOL = 1e-3
SEED = 0x5EED


@pytest.fixture(scope="module")
def torch_dev(pkg):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    pkg.init()
    return torch


def up(torch, arr):
    t = torch.from_numpy(np.ascontiguousarray(arr)).cuda()
    return t


def down(t):
    return t.cpu().numpy()


def stream(torch):
    return torch.cuda.current_stream().cuda_stream


def say(*a):
    print("[gpu case]", *a, flush=True)


def weights(pkg, dtype, rows, cols, mid=0, sigma=0.02):
    return pkg.synth_quantized(dtype, SEED ^ (7 << 32) ^ mid, sigma, rows, cols)


def acts(pkg, n, cols, mid=0):
    return pkg.fill_normal(SEED ^ 0xA11CE ^ mid, 1.0, n, cols)


# ------------------------------------------------------------------ dequant

def _same_bits(a, b):
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


@pytest.mark.parametrize("dtype,n", [(Q4_0, 32), (Q4_0, 4096 * 4096), (Q4_0, 1000), (Q4_0, 7),
                                     (Q8_0, 4096 * 1024), (Q8_0, 999),
                                     (Q4_K, 256), (Q4_K, 4096 * 1024), (Q4_K, 300)])
def test_dequant_bit_exact(pkg, orc, torch_dev, dtype, n):
    torch = torch_dev
    cols = 256 if dtype == Q4_K else 32
    blocks_n = (n + cols - 1) // cols * cols
    raw = weights(pkg, dtype, 1, blocks_n, mid=n)
    say("dequant", dtype, n)
    d_raw = up(torch, raw)
    d_out = torch.empty(n, dtype=torch.float32, device="cuda")
    pkg.qdequant(dtype, d_raw.data_ptr(), raw.size, d_out.data_ptr(), n, stream(torch))
    torch.cuda.synchronize()
    assert _same_bits(down(d_out), orc.dequantize(dtype, raw, n))


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
def test_dequant_random_bytes_bit_exact(pkg, orc, torch_dev, dtype):
    """Uniformly random block bytes: every f16 scale code (subnormal, inf,
    NaN) and every 6-bit scale/min code appear."""
    torch = torch_dev
    bs, ts = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144)}[dtype]
    nblk = 20000
    raw = np.random.default_rng(dtype).integers(0, 256, nblk * ts, dtype=np.uint8)
    n = nblk * bs
    say("dequant random bytes", dtype)
    d_raw = up(torch, raw)
    d_out = torch.empty(n, dtype=torch.float32, device="cuda")
    pkg.qdequant(dtype, d_raw.data_ptr(), raw.size, d_out.data_ptr(), n, stream(torch))
    torch.cuda.synchronize()
    assert _same_bits(down(d_out), orc.dequantize(dtype, raw, n))


def test_dequant_every_f16_scale(pkg, orc, torch_dev):
    """Q8_0 blocks with d = each of the 65536 f16 codes and q = 1: the device
    f16 decode equals the oracle's for every code."""
    torch = torch_dev
    codes = np.arange(65536, dtype=np.uint16)
    raw = np.zeros((65536, 34), dtype=np.uint8)
    raw[:, 0] = codes & 0xFF
    raw[:, 1] = codes >> 8
    raw[:, 2:] = 1
    raw = raw.reshape(-1)
    n = 65536 * 32
    say("dequant every f16 code")
    d_raw = up(torch, raw)
    d_out = torch.empty(n, dtype=torch.float32, device="cuda")
    pkg.qdequant(Q8_0, d_raw.data_ptr(), raw.size, d_out.data_ptr(), n, stream(torch))
    torch.cuda.synchronize()
    assert _same_bits(down(d_out), orc.dequantize(Q8_0, raw, n))


@pytest.mark.parametrize("dtype", [F16, BF16, F32])
def test_dequant_float_types(pkg, orc, torch_dev, dtype):
    torch = torch_dev
    n = 70001
    raw = np.random.default_rng(5).integers(0, 256, n * (4 if dtype == F32 else 2), dtype=np.uint8)
    d_raw = up(torch, raw)
    d_out = torch.empty(n, dtype=torch.float32, device="cuda")
    pkg.qdequant(dtype, d_raw.data_ptr(), raw.size, d_out.data_ptr(), n, stream(torch))
    torch.cuda.synchronize()
    assert _same_bits(down(d_out), orc.dequantize(dtype, raw, n))


# --------------------------------------------------------------------- GEMV

def _gemv_check(pkg, orc, torch, dtype, rows, cols, check_rows=None, mid=0):
    raw = weights(pkg, dtype, rows, cols, mid=mid)
    x = acts(pkg, 1, cols, mid=mid)[0]
    say("gemv", dtype, rows, cols)
    d_w, d_x = up(torch, raw), up(torch, x)
    d_y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    pkg.qgemv(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), rows, cols,
              stream(torch))
    torch.cuda.synchronize()
    y = down(d_y)
    assert np.all(np.isfinite(y))
    rb = pkg.row_bytes(dtype, cols)
    sel = check_rows if check_rows is not None else [(0, rows)]
    worst = 0.0
    for r0, r1 in sel:
        sub = raw[r0 * rb:r1 * rb]
        ref = orc.forward_linear(dtype, sub, x, r1 - r0, cols, 8)
        deq = orc.dequantize(dtype, sub, (r1 - r0) * cols).reshape(r1 - r0, cols)
        worst = max(worst, orc.normalized_error(y[r0:r1], ref, deq, x))
    assert worst <= TOL, worst
    return worst


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (37, 4096), (1, 256), (4096, 14336),
                                       (300, 28672), (64, 65536)])
def test_gemv_parity(pkg, orc, torch_dev, dtype, rows, cols):
    _gemv_check(pkg, orc, torch_dev, dtype, rows, cols)


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
@pytest.mark.parametrize("rows,cols", [(24, 65792), (9, 131072), (5, 262144)])
def test_gemv_parity_long_rows(pkg, orc, torch_dev, dtype, rows, cols):
    # rows of more than 65536 weights take the generic one-wave-per-row kernels
    _gemv_check(pkg, orc, torch_dev, dtype, rows, cols)


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("cols", [64, 320, 96, 4064])
def test_gemv_parity_small_blocks(pkg, orc, torch_dev, dtype, cols):
    # n_cols % 64 != 0 takes the generic one-block-per-lane kernel
    _gemv_check(pkg, orc, torch_dev, dtype, 129, cols)


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
@pytest.mark.parametrize("rows,cols", [(1, 4096), (3, 4096), (6, 4096), (4099, 4096),
                                       (6150, 4096), (5, 8192), (4097, 8192), (16387, 8192)])
def test_gemv_row_sets(pkg, orc, torch_dev, dtype, rows, cols):
    # Rows of at most 128 items run as several row sets per workgroup sharing
    # x (one-wave sets for K = 4096, two-wave sets with workgroup-uniform
    # trips for K = 8192); these row counts leave sets of the last
    # workgroups without a tile, or with one trip fewer than set 0.
    _gemv_check(pkg, orc, torch_dev, dtype, rows, cols, mid=rows)


@pytest.mark.parametrize("dtype", [Q4_0, Q4_K])
def test_gemv_8b_shapes_subsets(pkg, orc, torch_dev, dtype):
    for rows, cols in [(6144, 4096), (28672, 4096), (128256, 4096)]:
        _gemv_check(pkg, orc, torch_dev, dtype, rows, cols,
                    check_rows=[(0, 1024), (rows // 2, rows // 2 + 512), (rows - 1024, rows)])


@pytest.mark.parametrize("dtype", [Q8_0, Q4_0, Q4_K])
def test_gemv_linearity_full_lm_head(pkg, torch_dev, dtype):
    """Size-independent check at the full lm_head shape: W(2x) = 2 Wx exactly
    (the kernel's per-item scaling is a power of two), and W(x1 + x2) equals
    Wx1 + Wx2 up to the kernel's rounding of x to fp16 (2^-11 relative):
    normalized by ||W_r|| (||x1|| + ||x2||), within 1e-4."""
    torch = torch_dev
    rows, cols = 128256, 4096
    raw = weights(pkg, dtype, rows, cols, mid=99)
    x = acts(pkg, 2, cols, mid=99)
    say("gemv linearity lm_head", dtype)
    d_w = up(torch, raw)
    outs = []
    for v in (x[0], 2 * x[0], x[1], x[0] + x[1]):
        d_x = up(torch, v.astype(np.float32))
        d_y = torch.empty(rows, dtype=torch.float32, device="cuda")
        pkg.qgemv(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), rows, cols,
                  stream(torch))
        outs.append(down(d_y))
    # row norms of the dequantized weights (the device dequantizer is
    # bit-exact with the oracle's, checked above)
    d_deq = torch.empty(rows * cols, dtype=torch.float32, device="cuda")
    pkg.qdequant(dtype, d_w.data_ptr(), raw.size, d_deq.data_ptr(), rows * cols, stream(torch))
    wn = down(torch.linalg.vector_norm(d_deq.view(rows, cols).double(), dim=1))
    torch.cuda.synchronize()
    assert np.array_equal(outs[1], 2 * outs[0])
    xn = np.linalg.norm(x[0].astype(np.float64)) + np.linalg.norm(x[1].astype(np.float64))
    dev = np.abs(outs[3].astype(np.float64) - outs[0] - outs[2]) / (wn * xn)
    assert dev.max() <= 1e-4, dev.max()


def test_gemv_multi(pkg, orc, torch_dev):
    torch = torch_dev
    cols = 4096
    spec = [(Q4_0, 4096), (Q4_0, 1024), (Q4_0, 1024), (Q4_K, 333), (Q8_0, 77)]
    raws = [weights(pkg, dt, r, cols, mid=i) for i, (dt, r) in enumerate(spec)]
    x = acts(pkg, 1, cols, mid=5)[0]
    d_ws = [up(torch, r) for r in raws]
    d_ys = [torch.empty(r, dtype=torch.float32, device="cuda") for _, r in spec]
    d_x = up(torch, x)
    say("gemv multi")
    pkg.qgemv_multi([dt for dt, _ in spec], [t.data_ptr() for t in d_ws], [r.size for r in raws],
                    [r for _, r in spec], d_x.data_ptr(), [t.data_ptr() for t in d_ys], cols,
                    stream(torch))
    torch.cuda.synchronize()
    for (dt, r), raw, d_y in zip(spec, raws, d_ys):
        ref = orc.forward_linear(dt, raw, x, r, cols, 8)
        deq = orc.dequantize(dt, raw, r * cols).reshape(r, cols)
        assert orc.normalized_error(down(d_y), ref, deq, x) <= TOL


# ------------------------------------------------------------ small batch

@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
@pytest.mark.parametrize("n_tok", [1, 2, 4, 8, 16, 19, 33, 64, 70])
@pytest.mark.parametrize("rows,cols", [(1000, 4096), (256, 14336)])
def test_batched_parity(pkg, orc, torch_dev, errlog, dtype, n_tok, rows, cols):
    # 1 token: the decode GEMV; 2: the GEMV over both tokens, x rounded to
    # fp16; 4..64: the small-batch kernel (19 in two token groups of 16, 33
    # and 64 in four), x rounded to fp16; 70: the prefill GEMM on
    # bf16-rounded x
    torch = torch_dev
    raw = weights(pkg, dtype, rows, cols, mid=n_tok)
    xs = acts(pkg, n_tok, cols, mid=n_tok)
    say("batched", dtype, n_tok, rows, cols)
    d_w, d_x = up(torch, raw), up(torch, xs)
    d_y = torch.full((n_tok, rows), float("nan"), dtype=torch.float32, device="cuda")
    pkg.qgemv_batched(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), n_tok,
                      rows, cols, False, stream(torch))
    torch.cuda.synchronize()
    y = down(d_y)
    ref = orc.forward_linear_batch(dtype, raw, xs, rows, cols, 8)
    deq = orc.dequantize(dtype, raw, rows * cols).reshape(rows, cols)
    err = orc.normalized_error(y, ref, deq, xs)
    path = "gemv" if n_tok == 1 else "batched_f16" if n_tok <= 64 else "gemm_bf16"
    errlog(f"batched {dtype} n_tok={n_tok} {rows}x{cols}", err, path=path)
    assert err <= {"gemv": 1e-6, "batched_f16": 1e-4, "gemm_bf16": 4e-4}[path]


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
@pytest.mark.parametrize("n_tok,rows,cols", [(2, 77, 320), (5, 33, 64), (12, 16, 8192),
                                             (16, 3000, 1024), (3, 1, 2304)])
def test_batched_ragged(pkg, orc, torch_dev, dtype, n_tok, rows, cols):
    """Row counts that end inside a 16-row tile, K that ends inside a K
    group (Q4_K rounds cols up to its 256 block), single-row matrices."""
    torch = torch_dev
    if dtype == Q4_K:
        cols = (cols + 255) // 256 * 256
    raw = weights(pkg, dtype, rows, cols, mid=n_tok + 40)
    xs = acts(pkg, n_tok, cols, mid=n_tok + 40)
    say("batched ragged", dtype, n_tok, rows, cols)
    d_w, d_x = up(torch, raw), up(torch, xs)
    d_y = torch.full((n_tok, rows), float("nan"), dtype=torch.float32, device="cuda")
    pkg.qgemv_batched(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), n_tok,
                      rows, cols, False, stream(torch))
    torch.cuda.synchronize()
    ref = orc.forward_linear_batch(dtype, raw, xs, rows, cols, 8)
    deq = orc.dequantize(dtype, raw, rows * cols).reshape(rows, cols)
    assert orc.normalized_error(down(d_y), ref, deq, xs) <= TOL


def test_batched_repeat_bitwise(pkg, torch_dev):
    """Split-K tiles combine in a fixed order through per-tile counters that
    each launch leaves at zero: repeated calls, with other shapes (and a
    larger workspace) in between, give bit-identical results."""
    torch = torch_dev
    shapes = [(Q4_K, 16, 4096, 14336), (Q8_0, 7, 6144, 4096), (Q4_0, 16, 300, 4096),
              (Q6_K, 12, 4096, 14336)]
    first = []
    bufs = []
    for i, (dt, n_tok, rows, cols) in enumerate(shapes):
        raw = weights(pkg, dt, rows, cols, mid=90 + i)
        xs = acts(pkg, n_tok, cols, mid=90 + i)
        bufs.append((dt, n_tok, rows, cols, up(torch, raw), raw.size, up(torch, xs)))
    say("batched repeat", len(shapes))
    for rep in range(3):
        for j, (dt, n_tok, rows, cols, d_w, wl, d_x) in enumerate(bufs):
            d_y = torch.full((n_tok, rows), float("nan"), dtype=torch.float32, device="cuda")
            pkg.qgemv_batched(dt, d_w.data_ptr(), wl, d_x.data_ptr(), d_y.data_ptr(), n_tok, rows,
                              cols, False, stream(torch))
            torch.cuda.synchronize()
            y = down(d_y)
            assert np.isfinite(y).all()
            if rep == 0:
                first.append(y)
            else:
                assert np.array_equal(y.view(np.uint32), first[j].view(np.uint32)), (rep, j)


def test_batched_two_streams(pkg, torch_dev):
    """Matrices with few rows split K over workgroups through a workspace
    kept per (device, stream): calls queued on two streams at once give the
    same bits as the same calls run one after another on one stream."""
    torch = torch_dev
    # 40 and 64 tokens: token groups with K groups; the last two run the
    # GEMM route: bf16 x in one per-stream buffer, K pieces in the other
    cases = [(Q4_K, 16, 4096, 14336), (Q4_0, 8, 6144, 4096), (Q8_0, 12, 4096, 4096),
             (Q4_0, 40, 4096, 4096), (Q4_K, 64, 6144, 4096), (Q4_0, 80, 4096, 4096),
             (Q4_K, 96, 6144, 4096), (Q6_K, 32, 4096, 14336)]
    bufs = []
    for i, (dt, n_tok, rows, cols) in enumerate(cases):
        raw = weights(pkg, dt, rows, cols, mid=120 + i)
        xs = acts(pkg, n_tok, cols, mid=120 + i)
        bufs.append((dt, n_tok, rows, cols, up(torch, raw), raw.size, up(torch, xs)))
    say("batched two streams", len(cases))

    def run(b, d_y, s):
        dt, n_tok, rows, cols, d_w, wl, d_x = b
        pkg.qgemv_batched(dt, d_w.data_ptr(), wl, d_x.data_ptr(), d_y.data_ptr(), n_tok, rows,
                          cols, False, s)

    ref = []
    for b in bufs:
        d_y = torch.full((b[1], b[2]), float("nan"), dtype=torch.float32, device="cuda")
        run(b, d_y, stream(torch))
        torch.cuda.synchronize()
        ref.append(down(d_y))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()  # default priority
    outs = [[torch.full((b[1], b[2]), float("nan"), dtype=torch.float32, device="cuda")
             for b in bufs] for _ in range(2)]
    torch.cuda.synchronize()
    for rep in range(4):
        for j, b in enumerate(bufs):
            run(b, outs[0][j], s1.cuda_stream)
            run(bufs[-1 - j], outs[1][len(bufs) - 1 - j], s2.cuda_stream)
    torch.cuda.synchronize()
    for k in range(2):
        for j in range(len(bufs)):
            assert np.array_equal(down(outs[k][j]).view(np.uint32), ref[j].view(np.uint32)), (k, j)


@pytest.mark.parametrize("cols", [4096, 14336])
@pytest.mark.parametrize("n_tok", [1, 6, 40, 70])
def test_batched_accumulate(pkg, orc, torch_dev, cols, n_tok):
    """accumulate=1 is the kernel contract of fused_gemv_q4k_batched
    (out += W x, fused_gemv_q4k.rs:694); it keeps every pass, of one token
    or of more than 64 (passes of 64), on the small-batch kernel."""
    torch = torch_dev
    rows = 512
    raw = weights(pkg, Q4_K, rows, cols, mid=3)
    xs = acts(pkg, n_tok, cols, mid=3)
    base = np.random.default_rng(1).standard_normal((n_tok, rows)).astype(np.float32)
    d_w, d_x, d_y = up(torch, raw), up(torch, xs), up(torch, base)
    pkg.qgemv_batched(Q4_K, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), n_tok, rows,
                      cols, True, stream(torch))
    torch.cuda.synchronize()
    outs = base.copy()
    orc.fused_gemv_q4k_batched(raw, xs, outs, rows, cols)
    deq = orc.dequantize(Q4_K, raw, rows * cols).reshape(rows, cols)
    assert orc.normalized_error(down(d_y), outs, deq, xs) <= TOL


# ------------------------------------------------------------ prefill GEMM

@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
@pytest.mark.parametrize("m,rows,cols", [(512, 4096, 4096), (77, 300, 1024), (2048, 512, 4096),
                                         (256, 1024, 14336)])
def test_gemm_bf16_parity(pkg, orc, torch_dev, dtype, m, rows, cols):
    torch = torch_dev
    raw = weights(pkg, dtype, rows, cols, mid=m)
    x = acts(pkg, m, cols, mid=m)
    xb = pkg.to_bf16_bits(x)
    x_fed = (xb.astype(np.uint32) << 16).view(np.float32)
    say("gemm bf16", dtype, m, rows, cols)
    d_w, d_x = up(torch, raw), up(torch, xb.view(np.int16))
    d_y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
    pkg.qgemm(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), BF16, d_y.data_ptr(), m, rows,
              cols, stream(torch))
    torch.cuda.synchronize()
    y = down(d_y)
    assert np.all(np.isfinite(y))
    toks = sorted(set([0, 1, m // 2, m - 1] + list(range(max(0, m - 3), m))))
    ref = orc.forward_linear_batch(dtype, raw, x_fed[toks], rows, cols, 8)
    deq = orc.dequantize(dtype, raw, rows * cols).reshape(rows, cols)
    assert orc.normalized_error(y[toks], ref, deq, x_fed[toks]) <= TOL


# Every work decomposition of the bf16 GEMM, on both routes (forced per
# call with SWAMP_GEMM_ROUTE).  Fused kernel (256-token x 256-row tiles on
# the CUs of one MI355X): complete rounds of full tiles; full tiles plus a
# last round of 128-token half tiles (ragged tokens and rows: the second
# half of the short last token tile is empty); one partial round of full
# tiles; at most half a round: full tiles in 2 and in 5 K pieces summed
# through the workspace; short K (8 steps): half tiles; at most 64 tokens:
# quarter tiles, split along K.  Dequantize-once route (plain bf16 GEMM):
# full rounds plus a last round of half tiles (1900 x 28572), 192-row tiles
# (2048 x 6144), 128-row tiles (2048 x 4096 x 14336, 100 x 600), 128-row
# tiles split along K into 8 pieces (64 x 4096 x 14336) and 2 (1 x 600).
DECOMP_CASES = [(2048, 8192, 4096), (1900, 28572, 4096), (2048, 6144, 4096), (2048, 4096, 14336),
                (512, 6144, 4096), (100, 600, 512), (48, 28672, 4096), (64, 4096, 14336), (1, 600, 1024)]


@pytest.mark.parametrize("route", ["fused", "dq"])
@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
@pytest.mark.parametrize("m,rows,cols", DECOMP_CASES)
def test_gemm_bf16_decompositions(pkg, orc, torch_dev, monkeypatch, dtype, m, rows, cols, route):
    torch = torch_dev
    monkeypatch.setenv("SWAMP_GEMM_ROUTE", route)
    raw = weights(pkg, dtype, rows, cols, mid=rows ^ m)
    x = acts(pkg, m, cols, mid=m ^ cols)
    xb = pkg.to_bf16_bits(x)
    x_fed = (xb.astype(np.uint32) << 16).view(np.float32)
    say("gemm bf16 decomposition", route, dtype, m, rows, cols)
    d_w, d_x = up(torch, raw), up(torch, xb.view(np.int16))
    d_y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
    pkg.qgemm(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), BF16, d_y.data_ptr(), m, rows,
              cols, stream(torch))
    torch.cuda.synchronize()
    y = down(d_y)
    assert np.all(np.isfinite(y))
    # tokens at tile and half-tile edges, rows at both ends and the middle
    toks = sorted(set(k for k in [0, 127, 128, 255, 256, m // 2, m - 129, m - 128, m - 1]
                      if 0 <= k < m))
    rb = pkg.row_bytes(dtype, cols)
    for r0, r1 in [(0, 384), (rows // 2 - 128, rows // 2 + 128), (rows - 300, rows)]:
        sub = raw[r0 * rb:r1 * rb]
        ref = orc.forward_linear_batch(dtype, sub, x_fed[toks], r1 - r0, cols, 8)
        deq = orc.dequantize(dtype, sub, (r1 - r0) * cols).reshape(r1 - r0, cols)
        assert orc.normalized_error(y[toks, r0:r1], ref, deq, x_fed[toks]) <= TOL, (r0, r1)


def test_gemm_rows_tail_and_token_consistency(pkg, orc, torch_dev):
    """GEMM token rows equal the per-token GEMV within tolerance; a ragged
    row count (not a tile multiple) leaves no NaN."""
    torch = torch_dev
    m, rows, cols = 300, 777, 2048
    raw = weights(pkg, Q4_0, rows, cols, mid=42)
    x = acts(pkg, m, cols, mid=42)
    xb = pkg.to_bf16_bits(x)
    x_fed = (xb.astype(np.uint32) << 16).view(np.float32)
    d_w, d_x = up(torch, raw), up(torch, xb.view(np.int16))
    d_y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
    pkg.qgemm(Q4_0, d_w.data_ptr(), raw.size, d_x.data_ptr(), BF16, d_y.data_ptr(), m, rows, cols,
              stream(torch))
    d_xf = up(torch, x_fed[m - 1])
    d_g = torch.empty(rows, dtype=torch.float32, device="cuda")
    pkg.qgemv(Q4_0, d_w.data_ptr(), raw.size, d_xf.data_ptr(), d_g.data_ptr(), rows, cols,
              stream(torch))
    torch.cuda.synchronize()
    y = down(d_y)
    assert np.all(np.isfinite(y))
    g = down(d_g)
    # both paths are within the contract of the same exact product, so they
    # agree to twice the normalized tolerance
    deq = orc.dequantize(Q4_0, raw, rows * cols).reshape(rows, cols)
    assert orc.normalized_error(y[m - 1], g, deq, x_fed[m - 1]) <= 2 * TOL


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
@pytest.mark.parametrize("m,rows,cols", [(512, 4096, 4096), (77, 300, 1024), (2048, 512, 4096),
                                         (256, 1024, 14336), (1, 33, 128), (130, 200, 768)])
def test_gemm_int8_parity(pkg, orc, torch_dev, dtype, m, rows, cols):
    """int8 matrix-core GEMM against Q8_0 activations: x is quantized on the
    device (swamp_quantize_q8_0, byte-identical to the host quantizer), and
    the oracle multiplies the dequantized Q8_0 activations -- the values the
    kernel actually consumed.  Q4_K rows are whole 256-weight super-blocks;
    768 columns are 6 K steps of 128, three super-blocks."""
    if dtype == Q4_K and cols % 256:
        pytest.skip("Q4_K rows are whole 256-weight super-blocks")
    torch = torch_dev
    raw = weights(pkg, dtype, rows, cols, mid=m + 5)
    x = acts(pkg, m, cols, mid=m + 5)
    say("gemm int8", dtype, m, rows, cols)
    d_w, d_x = up(torch, raw), up(torch, x)
    d_q = torch.empty(m * cols // 32 * 34, dtype=torch.uint8, device="cuda")
    pkg.quantize_q8_0(d_x.data_ptr(), F32, d_q.data_ptr(), m * cols, stream(torch))
    d_y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
    pkg.qgemm(dtype, d_w.data_ptr(), raw.size, d_q.data_ptr(), Q8_0, d_y.data_ptr(), m, rows,
              cols, stream(torch))
    torch.cuda.synchronize()
    y = down(d_y)
    assert np.all(np.isfinite(y))
    xq = pkg.quantize(Q8_0, x)
    assert np.array_equal(down(d_q), xq)
    x_fed = orc.dequantize(Q8_0, xq, m * cols).reshape(m, cols)
    toks = sorted(set([0, m // 2, m - 1] + list(range(max(0, m - 3), m))))
    ref = orc.forward_linear_batch(dtype, raw, x_fed[toks], rows, cols, 8)
    deq = orc.dequantize(dtype, raw, rows * cols).reshape(rows, cols)
    assert orc.normalized_error(y[toks], ref, deq, x_fed[toks]) <= TOL


def test_gemm_int8_argument_errors(pkg, torch_dev):
    torch = torch_dev
    rows, cols, m = 64, 192, 8   # 192 is a multiple of 64 but not of 128
    raw = weights(pkg, Q4_0, rows, cols)
    d_w = up(torch, raw)
    d_q = torch.zeros(m * cols // 32 * 34, dtype=torch.uint8, device="cuda")
    d_y = torch.zeros((m, rows), dtype=torch.float32, device="cuda")
    with pytest.raises(pkg.GpuError) as e:
        pkg.qgemm(Q4_0, d_w.data_ptr(), raw.size, d_q.data_ptr(), Q8_0, d_y.data_ptr(), m, rows,
                  cols, stream(torch))
    assert e.value.code == pkg.ESHAPE
    rawk = weights(pkg, Q6_K, rows, 512)
    d_wk = up(torch, rawk)
    with pytest.raises(pkg.GpuError) as e:
        pkg.qgemm(Q6_K, d_wk.data_ptr(), rawk.size, d_q.data_ptr(), Q8_0, d_y.data_ptr(), m,
                  rows, 512, stream(torch))
    assert e.value.code == pkg.EDTYPE
    torch.cuda.synchronize()
    assert np.all(down(d_y) == 0)  # nothing written on error


# ------------------------------------------------------ activation quantizer

@pytest.mark.parametrize("x_type", [F32, BF16])
def test_quantize_q8_0_matches_host(pkg, torch_dev, x_type):
    torch = torch_dev
    n = 4096 * 33
    x = acts(pkg, 1, n, mid=8)[0]
    if x_type == BF16:
        xb = pkg.to_bf16_bits(x)
        x = (xb.astype(np.uint32) << 16).view(np.float32)
        d_x = up(torch, xb.view(np.int16))
    else:
        d_x = up(torch, x)
    d_q = torch.empty(n // 32 * 34, dtype=torch.uint8, device="cuda")
    pkg.quantize_q8_0(d_x.data_ptr(), x_type, d_q.data_ptr(), n, stream(torch))
    torch.cuda.synchronize()
    host = pkg.quantize(Q8_0, x.reshape(1, -1))
    assert np.array_equal(down(d_q), host)


@pytest.mark.parametrize("x_type", [F32, BF16])
@pytest.mark.parametrize("n_blocks,q_offset", [(1, 0), (7, 0), (13, 0), (8 * 37 + 5, 0),
                                                (8 * 37 + 5, 2), (8 * 64, 1)])
def test_quantize_q8_0_tails_and_alignment(pkg, torch_dev, x_type, n_blocks, q_offset):
    """Block counts that leave a partial group of 8 (whole groups go to the
    vector kernel, the rest one element per thread), and an output buffer
    that is not 4-byte aligned (every block on the byte-store kernel).  The
    input holds an all-zero block, a block of subnormal-sized values, large
    values and ties at .5 after scaling."""
    torch = torch_dev
    n = 32 * n_blocks
    x = acts(pkg, 1, n, mid=9 + n_blocks)[0].copy()
    x[:32] = 0.0
    if n_blocks > 2:
        x[32:64] *= 1e-30
        x[64:96] = np.linspace(-3e4, 3e4, 32, dtype=np.float32)
    if x_type == BF16:
        xb = pkg.to_bf16_bits(x)
        x = (xb.astype(np.uint32) << 16).view(np.float32)
        d_x = up(torch, xb.view(np.int16))
    else:
        d_x = up(torch, x)
    buf = torch.full((n_blocks * 34 + 8,), 0xA5, dtype=torch.uint8, device="cuda")
    pkg.quantize_q8_0(d_x.data_ptr(), x_type, buf.data_ptr() + q_offset, n, stream(torch))
    torch.cuda.synchronize()
    got = down(buf)
    host = pkg.quantize(Q8_0, x.reshape(1, -1))
    assert np.array_equal(got[q_offset:q_offset + n_blocks * 34], host)
    assert np.all(got[:q_offset] == 0xA5) and np.all(got[q_offset + n_blocks * 34:] == 0xA5)


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
def test_empty_and_zero_k_calls(pkg, torch_dev, dtype):
    """Calls with no rows or no tokens return OK and leave y alone; calls with
    K = 0 write the empty sums (zeros) over y, and the accumulating batched
    form adds nothing (linear.rs:184 returns on an empty batch).  The
    arguments are still validated first (the weight length covers the shape)."""
    torch = torch_dev
    s = stream(torch)
    d_w = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    d_x = torch.ones(4096, dtype=torch.float32, device="cuda")
    d_q = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    d_y = torch.full((64,), 7.0, dtype=torch.float32, device="cuda")

    def y_is(v):
        torch.cuda.synchronize()
        return bool(torch.all(d_y == v).item())

    wp, xp, yp = d_w.data_ptr(), d_x.data_ptr(), d_y.data_ptr()
    wl = d_w.numel()  # enough bytes for every shape below
    pkg.qgemv(dtype, wp, wl, xp, yp, 0, 256, s)
    pkg.qgemv_batched(dtype, wp, wl, xp, yp, 0, 4, 256, 0, s)
    pkg.qgemv_batched(dtype, wp, wl, xp, yp, 4, 0, 256, 0, s)
    pkg.qgemm(dtype, wp, wl, xp, BF16, yp, 0, 8, 256, s)
    pkg.qgemm(dtype, wp, wl, d_q.data_ptr(), Q8_0, yp, 8, 0, 256, s)
    pkg.quantize_q8_0(xp, F32, d_q.data_ptr(), 0, s)
    pkg.qdequant(dtype, wp, wl, yp, 0, s)
    assert y_is(7.0)
    pkg.qgemv_batched(dtype, wp, wl, xp, yp, 4, 8, 0, 1, s)  # accumulate over K = 0
    assert y_is(7.0)
    pkg.qgemv(dtype, wp, wl, xp, yp, 64, 0, s)
    assert y_is(0.0)
    d_y.fill_(7.0)
    pkg.qgemv_batched(dtype, wp, wl, xp, yp, 4, 16, 0, 0, s)
    assert y_is(0.0)
    d_y.fill_(7.0)
    pkg.qgemm(dtype, wp, wl, xp, BF16, yp, 8, 8, 0, s)
    assert y_is(0.0)
    d_y.fill_(7.0)
    pkg.qgemm(dtype, wp, wl, d_q.data_ptr(), Q8_0, yp, 4, 16, 0, s)
    assert y_is(0.0)


# ------------------------------------------------------------ legacy exports

def test_legacy_fused_gemv_q4k_host_pointers(pkg, orc, torch_dev):
    rows, cols = 333, 2048
    raw = weights(pkg, Q4_K, rows, cols, mid=11)
    x = acts(pkg, 1, cols, mid=11)[0]
    out = np.full(rows, 5.0, np.float32)
    pkg.gpu_lib().swamp_fused_gemv_q4k(raw.ctypes.data, x.ctypes.data, out.ctypes.data, rows, cols)
    ref = orc.fused_gemv_q4k(raw, x, rows, cols)
    deq = orc.dequantize(Q4_K, raw, rows * cols).reshape(rows, cols)
    assert orc.normalized_error(out, ref, deq, x) <= TOL


def test_legacy_gemv_q8_vnni_kat(pkg, orc, fixtures, torch_dev):
    L = pkg.gpu_lib()
    for t in fixtures["int8_dot_kat"]:
        w = np.array(t["w"], dtype=np.int8)
        a = np.array(t["a"], dtype=np.int8)
        got = L.swamp_gemv_q8_vnni(w.ctypes.data, a.ctypes.data, t["k"], 1.0)
        assert got == float(np.float32(t["dot"]))
        assert L.swamp_gemv_q8_vnni(w.ctypes.data, a.ctypes.data, t["k"], 0.5) == \
            orc.gemv_q8_dot(w, a, 0.5)


# ------------------------------------------------------------------ GGUF

def test_gguf_upload_then_gemv(pkg, orc, torch_dev, tmp_path):
    """The input side of the path end to end: weights written into a GGUF
    file, read back by the mapped reader (include/swamp_gguf.h), copied to
    the device by swamp_gguf_upload and multiplied by swamp_qgemv; the
    oracle multiplies the same bytes taken from the file."""
    import sys, os
    sys.path.insert(0, os.path.dirname(__file__))
    from gguf_writer import STRING, write_gguf
    torch = torch_dev
    rows, cols = 700, 4096
    mats = {"blk.0.attn_q.weight": Q4_0, "blk.0.ffn_down.weight": Q8_0, "output.weight": Q4_K}
    raws = {n: weights(pkg, dt, rows, cols, mid=60 + i) for i, (n, dt) in enumerate(mats.items())}
    path = str(tmp_path / "model.gguf")
    write_gguf(path, [(n, [cols, rows], dt, raws[n].tobytes()) for n, dt in mats.items()],
               [("general.architecture", STRING, "llama")])
    x = acts(pkg, 1, cols, mid=61)[0]
    d_x = up(torch, x)
    say("gguf upload + gemv", rows, cols)
    with pkg.GgufFile(path) as g:
        for name, dt in mats.items():
            info = g.tensor_or_err(name)
            assert info.dtype == dt and info.shape == [cols, rows]
            d_w = torch.zeros(info.nbytes, dtype=torch.uint8, device="cuda")
            g.upload(info, d_w.data_ptr(), d_w.numel(), stream(torch))
            with pytest.raises(pkg.GpuError) as e:  # destination too small
                g.upload(info, d_w.data_ptr(), info.nbytes - 1, stream(torch))
            assert e.value.code == pkg.ESHAPE
            host = g.tensor_raw_bytes(info)
            assert np.array_equal(down(d_w), host)
            d_y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
            pkg.qgemv(dt, d_w.data_ptr(), d_w.numel(), d_x.data_ptr(), d_y.data_ptr(), info.shape[1],
                      info.shape[0], stream(torch))
            torch.cuda.synchronize()
            ref = orc.forward_linear(dt, host, x, rows, cols, 8)
            deq = orc.dequantize(dt, host, rows * cols).reshape(rows, cols)
            assert orc.normalized_error(down(d_y), ref, deq, x) <= TOL


def test_gemv_many(pkg, orc, torch_dev, errlog):
    """forward_gemvs (linear.rs:278-333): several GEMVs with their own x and
    shapes in one call, each written over its y; Q4_K and Q6_K as the
    reference handles them, plus Q4_0 and Q8_0."""
    torch = torch_dev
    spec = [(Q4_K, 3000, 4096), (14, 700, 14336), (Q4_0, 4096, 1024), (Q8_0, 33, 64),
            (Q4_K, 5, 256)]
    raws = [weights(pkg, dt, r, c, mid=200 + i) for i, (dt, r, c) in enumerate(spec)]
    xs = [acts(pkg, 1, c, mid=200 + i)[0] for i, (_, _, c) in enumerate(spec)]
    d_ws = [up(torch, r) for r in raws]
    d_xs = [up(torch, x) for x in xs]
    d_ys = [torch.full((r,), float("nan"), dtype=torch.float32, device="cuda") for _, r, _ in spec]
    say("gemv many", len(spec))
    pkg.qgemv_many([dt for dt, _, _ in spec], [t.data_ptr() for t in d_ws],
                   [r.size for r in raws], [r for _, r, _ in spec], [c for _, _, c in spec],
                   [t.data_ptr() for t in d_xs], [t.data_ptr() for t in d_ys], stream(torch))
    torch.cuda.synchronize()
    for (dt, r, c), raw, x, d_y in zip(spec, raws, xs, d_ys):
        ref = orc.forward_linear(dt, raw, x, r, c, 8)
        deq = orc.dequantize(dt, raw, r * c).reshape(r, c)
        err = errlog(f"gemv many dtype={dt} {r}x{c}", orc.normalized_error(down(d_y), ref, deq, x),
                     path="gemv")
        assert err <= 1e-6
    # a bad spec anywhere: nothing is launched
    d_y0 = torch.full((spec[0][1],), 7.0, dtype=torch.float32, device="cuda")
    with pytest.raises(pkg.GpuError):
        pkg.qgemv_many([Q4_K, Q4_K], [d_ws[0].data_ptr(), d_ws[0].data_ptr()],
                       [raws[0].size, 10], [spec[0][1], spec[0][1]], [4096, 4096],
                       [d_xs[0].data_ptr()] * 2, [d_y0.data_ptr(), d_y0.data_ptr()],
                       stream(torch))
    torch.cuda.synchronize()
    assert bool((d_y0 == 7.0).all())
