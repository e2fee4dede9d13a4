"""GPU parity of the Q6_K entry points against the CPU oracle (dequant_q6k,
swamp-gguf/src/quant/q6_k.rs:7-56; fused_gemv_q6k scalar body,
swamp-kernels/src/fused_gemv_q6k.rs:248-291; the Q6_K arms of forward_linear,
forward_linear_multi and fallback_gemv, swamp-engine/src/linear.rs:48-66,
128-144, 336-364).  Gates: dequantization bit-identical; GEMV outputs within
max_r |y - y_ref| / (||W_r|| ||x||) <= 1e-3."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_K, Q6_K = 12, 14
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
    return torch.from_numpy(np.ascontiguousarray(arr)).cuda()


def down(t):
    return t.cpu().numpy()


def stream(torch):
    return torch.cuda.current_stream().cuda_stream


def say(*a):
    print("[gpu case]", *a, flush=True)


def weights(pkg, dtype, rows, cols, mid=0):
    return pkg.synth_quantized(dtype, SEED ^ (9 << 32) ^ mid, 0.02, rows, cols)


def acts(pkg, n, cols, mid=0):
    return pkg.fill_normal(SEED ^ 0xB0B ^ mid, 1.0, n, cols)


def _same_bits(a, b):
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


# ------------------------------------------------------------------ dequant

@pytest.mark.parametrize("n", [256, 300, 7, 4096 * 1024])
def test_q6k_dequant_bit_exact(pkg, orc, torch_dev, n):
    torch = torch_dev
    raw = weights(pkg, Q6_K, 1, (n + 255) // 256 * 256, mid=n)
    say("q6k dequant", n)
    d_raw = up(torch, raw)
    d_out = torch.empty(n, dtype=torch.float32, device="cuda")
    pkg.qdequant(Q6_K, d_raw.data_ptr(), raw.size, d_out.data_ptr(), n, stream(torch))
    torch.cuda.synchronize()
    assert _same_bits(down(d_out), orc.dequantize(Q6_K, raw, n))


def test_q6k_dequant_random_bytes_2_byte_offset(pkg, orc, torch_dev):
    """Uniformly random blocks (every f16 d code class: zero, subnormal,
    inf, NaN; every int8 scale) read from a base 2 bytes past a 4-byte
    boundary (the block size 210 keeps blocks 2-byte aligned only)."""
    torch = torch_dev
    nblk = 20000
    raw = np.random.default_rng(14).integers(0, 256, nblk * 210, dtype=np.uint8)
    n = nblk * 256
    say("q6k dequant random bytes")
    d_buf = up(torch, np.concatenate([np.zeros(2, np.uint8), raw]))
    d_out = torch.empty(n, dtype=torch.float32, device="cuda")
    pkg.qdequant(Q6_K, d_buf.data_ptr() + 2, raw.size, d_out.data_ptr(), n, stream(torch))
    torch.cuda.synchronize()
    assert _same_bits(down(d_out), orc.dequantize(Q6_K, raw, n))


# --------------------------------------------------------------------- GEMV

def _gemv(pkg, torch, raw, x, rows, cols):
    d_w, d_x = up(torch, raw), up(torch, x)
    d_y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    pkg.qgemv(Q6_K, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), rows, cols,
              stream(torch))
    torch.cuda.synchronize()
    return down(d_y)


def _check(pkg, orc, raw, x, y, rows, cols, sel=None):
    assert np.all(np.isfinite(y))
    rb = pkg.row_bytes(Q6_K, cols)
    worst = 0.0
    for r0, r1 in sel or [(0, rows)]:
        sub = raw[r0 * rb:r1 * rb]
        ref = orc.forward_linear(Q6_K, sub, x, r1 - r0, cols, 8)
        deq = orc.dequantize(Q6_K, sub, (r1 - r0) * cols).reshape(r1 - r0, cols)
        worst = max(worst, orc.normalized_error(y[r0:r1], ref, deq, x))
    assert worst <= TOL, worst
    return worst


# item kernel: n_cols % 512 == 0 and n_cols <= 65536 (one item per lane up
# to 32768, two beyond); generic kernel: odd block counts and longer rows
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (37, 4096), (1, 512), (4096, 14336),
                                       (300, 28672), (64, 36864), (33, 65536),
                                       (129, 256), (77, 1280), (16, 66048)])
def test_q6k_gemv_parity(pkg, orc, torch_dev, rows, cols):
    raw = weights(pkg, Q6_K, rows, cols, mid=rows ^ cols)
    x = acts(pkg, 1, cols, mid=cols)[0]
    say("q6k gemv", rows, cols)
    y = _gemv(pkg, torch_dev, raw, x, rows, cols)
    _check(pkg, orc, raw, x, y, rows, cols)


def test_q6k_gemv_lm_head_subsets_and_linearity(pkg, orc, torch_dev):
    """Llama-3 8B lm_head (128256 x 4096, Q6_K in Q4_K_M files): oracle on
    three row ranges; W(2x) = 2 Wx exactly on every row (per-item scaling is
    a power of two)."""
    torch = torch_dev
    rows, cols = 128256, 4096
    raw = weights(pkg, Q6_K, rows, cols, mid=1)
    x = acts(pkg, 1, cols, mid=1)[0]
    say("q6k gemv lm_head")
    y = _gemv(pkg, torch, raw, x, rows, cols)
    _check(pkg, orc, raw, x, y, rows, cols,
           sel=[(0, 1024), (rows // 2, rows // 2 + 512), (rows - 1024, rows)])
    y2 = _gemv(pkg, torch, raw, 2 * x, rows, cols)
    assert np.array_equal(y2, 2 * y)


def test_q6k_gemv_signed_scales_and_extreme_x(pkg, orc, torch_dev):
    """Random ql/qh/scale bytes with finite normal and subnormal d, and x
    spanning 2^-60 .. 2^60 across items."""
    torch = torch_dev
    rows, cols = 64, 4096
    rng = np.random.default_rng(5)
    blocks = rng.integers(0, 256, (rows * cols // 256, 210), dtype=np.uint8)
    d = np.where(rng.random(len(blocks)) < 0.5, rng.integers(0x0001, 0x0400, len(blocks)),
                 rng.integers(0x0400, 0x5000, len(blocks))).astype(np.uint16)
    d |= (rng.integers(0, 2, len(blocks)) << 15).astype(np.uint16)
    blocks[:, 208] = d & 0xFF
    blocks[:, 209] = d >> 8
    raw = blocks.reshape(-1)
    x = acts(pkg, 1, cols, mid=3)[0]
    x *= np.exp2(rng.integers(-60, 61, cols // 64).repeat(64)).astype(np.float32)
    say("q6k gemv random bytes")
    y = _gemv(pkg, torch, raw, x, rows, cols)
    _check(pkg, orc, raw, x, y, rows, cols)


def test_q6k_multi_mixed_with_q4k(pkg, orc, torch_dev):
    """forward_linear_multi with Q4_K and Q6_K matrices sharing x (both arms,
    linear.rs:108-144): each output equals its single GEMV."""
    torch = torch_dev
    for cols in (4096, 1280):
        spec = [(Q4_K, 512), (Q6_K, 1024), (Q6_K, 77), (Q4_K, 33)]
        raws = [weights(pkg, dt, r, cols, mid=i) for i, (dt, r) in enumerate(spec)]
        x = acts(pkg, 1, cols, mid=7)[0]
        d_ws = [up(torch, r) for r in raws]
        d_ys = [torch.empty(r, dtype=torch.float32, device="cuda") for _, r in spec]
        d_x = up(torch, x)
        say("q6k multi", cols)
        pkg.qgemv_multi([dt for dt, _ in spec], [t.data_ptr() for t in d_ws],
                        [r.size for r in raws], [r for _, r in spec], d_x.data_ptr(),
                        [t.data_ptr() for t in d_ys], cols, stream(torch))
        torch.cuda.synchronize()
        for (dt, r), raw, d_y in zip(spec, raws, d_ys):
            ref = orc.forward_linear(dt, raw, x, r, cols, 8)
            deq = orc.dequantize(dt, raw, r * cols).reshape(r, cols)
            assert orc.normalized_error(down(d_y), ref, deq, x) <= TOL, (dt, r, cols)


def _batched(pkg, torch, raw, xs, rows, cols, accumulate=False, base=None):
    n_tok = xs.shape[0]
    d_w, d_x = up(torch, raw), up(torch, xs)
    if base is None:
        d_y = torch.full((n_tok, rows), float("nan"), dtype=torch.float32, device="cuda")
    else:
        d_y = up(torch, base)
    pkg.qgemv_batched(Q6_K, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), n_tok,
                      rows, cols, accumulate, stream(torch))
    torch.cuda.synchronize()
    return down(d_y)


def _batched_err(pkg, orc, raw, xs, y, rows, cols, sel=None):
    rb = pkg.row_bytes(Q6_K, cols)
    worst = 0.0
    for r0, r1 in sel or [(0, rows)]:
        sub = raw[r0 * rb:r1 * rb]
        ref = orc.forward_linear_batch(Q6_K, sub, xs, r1 - r0, cols, 8)
        deq = orc.dequantize(Q6_K, sub, (r1 - r0) * cols).reshape(r1 - r0, cols)
        worst = max(worst, orc.normalized_error(y[:, r0:r1], ref, deq, xs))
    return worst


# passes on the matrix cores for rows of a multiple of 512 weights: up to 32
# tokens each (3..4 tokens, 5..8, 9..16, 17..32 in two token groups), K
# groups (1024 x 14336), K phases (32 tokens x 14336), a 70-token call in
# three passes (32 + 32 + 6), one block pair per row (512); two tokens run
# the GEMV over both; one token and rows of an odd number of blocks (768)
# run the decode GEMV per token
@pytest.mark.parametrize("n_tok,rows,cols", [(1, 300, 4096), (2, 77, 512), (2, 16385, 512), (5, 1000, 4096),
                                             (16, 1024, 14336), (17, 64, 14336),
                                             (32, 2000, 4096), (32, 100, 14336),
                                             (70, 256, 2048), (3, 40, 768), (5, 33, 512),
                                             (9, 200, 1024), (2, 40, 768)])
def test_q6k_batched(pkg, orc, torch_dev, errlog, n_tok, rows, cols):
    """forward_linear_batch on Q6_K, written over y (linear.rs:336-364):
    within the batched fp16 bound (1e-4; x and the weights rounded to fp16
    once) against the oracle's per-token GEMV; the one-token pass and the
    odd-block rows are swamp_qgemv bit for bit; accumulate is refused."""
    torch = torch_dev
    raw = weights(pkg, Q6_K, rows, cols, mid=n_tok ^ rows)
    xs = acts(pkg, n_tok, cols, mid=n_tok)
    say("q6k batched", n_tok, rows, cols)
    y = _batched(pkg, torch, raw, xs, rows, cols)
    assert np.all(np.isfinite(y))
    err = errlog(f"q6k batched n_tok={n_tok} {rows}x{cols}",
                 _batched_err(pkg, orc, raw, xs, y, rows, cols), path="batched_f16")
    per_token = n_tok == 1 or cols % 512 != 0
    assert err <= (1e-5 if per_token else 1e-4)
    if per_token:
        for t in range(n_tok):
            assert np.array_equal(_gemv(pkg, torch, raw, xs[t], rows, cols), y[t])
    d_w, d_x = up(torch, raw), up(torch, xs)
    d_y = torch.zeros((n_tok, rows), dtype=torch.float32, device="cuda")
    with pytest.raises(pkg.GpuError) as e:
        pkg.qgemv_batched(Q6_K, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), n_tok,
                          rows, cols, True, stream(torch))
    assert e.value.code == pkg.EDTYPE


@pytest.mark.parametrize("n_tok", [2, 4, 16, 32])
def test_q6k_batched_lm_head_subsets(pkg, orc, torch_dev, errlog, n_tok):
    """Llama-3 8B lm_head, 128256 x 4096 Q6_K (as Q4_K_M files keep it), in
    one pass: the oracle on three row ranges; every token's rows equal the
    same call's rows with the tokens reversed (the pass is per-token exact
    in its order of sums, whatever the token's slot)."""
    torch = torch_dev
    rows, cols = 128256, 4096
    raw = weights(pkg, Q6_K, rows, cols, mid=3)
    xs = acts(pkg, n_tok, cols, mid=n_tok + 100)
    say("q6k batched lm_head", n_tok)
    y = _batched(pkg, torch, raw, xs, rows, cols)
    assert np.all(np.isfinite(y))
    sel = [(0, 512), (rows // 2, rows // 2 + 256), (rows - 512, rows)]
    err = errlog(f"q6k batched lm_head n_tok={n_tok}",
                 _batched_err(pkg, orc, raw, xs, y, rows, cols, sel=sel), path="batched_f16")
    assert err <= 1e-4
    y_rev = _batched(pkg, torch, raw, np.ascontiguousarray(xs[::-1]), rows, cols)
    assert np.array_equal(y_rev[::-1], y)


def test_q6k_gguf_upload_then_gemv(pkg, orc, torch_dev, tmp_path):
    from gguf_writer import write_gguf
    torch = torch_dev
    rows, cols = 96, 4096
    raw = weights(pkg, Q6_K, rows, cols, mid=11)
    path = str(tmp_path / "q6k.gguf")
    write_gguf(path, [("output.weight", [cols, rows], Q6_K, raw.tobytes())])
    x = acts(pkg, 1, cols, mid=11)[0]
    with pkg.GgufFile(path) as g:
        info = g.tensor("output.weight")
        assert info.dtype == Q6_K and info.nbytes == raw.size
        d_w = torch.empty(info.nbytes, dtype=torch.uint8, device="cuda")
        g.upload(info, d_w.data_ptr(), d_w.numel(), stream(torch))
    d_x = up(torch, x)
    d_y = torch.empty(rows, dtype=torch.float32, device="cuda")
    say("q6k gguf upload gemv")
    pkg.qgemv(Q6_K, d_w.data_ptr(), d_w.numel(), d_x.data_ptr(), d_y.data_ptr(), rows, cols,
              stream(torch))
    torch.cuda.synchronize()
    _check(pkg, orc, raw, x, down(d_y), rows, cols)


# ------------------------------------------------------------ prefill GEMM

@pytest.mark.parametrize("m,rows,cols", [(64, 1000, 4096), (300, 4096, 14336), (2048, 2048, 4096),
                                         (7, 333, 1280)])
def test_q6k_gemm_bf16(pkg, orc, torch_dev, errlog, m, rows, cols):
    """Q6_K prefill GEMM (bf16 x): the weights dequantized once to bf16 (the
    dequantizer's exact values, rounded to nearest even) and multiplied by
    the library GEMM; against forward_linear's Q6_K arm per token on the
    bf16-rounded x, within the contract (the Q4_K_M lm_head's prefill)."""
    torch = torch_dev
    raw = weights(pkg, Q6_K, rows, cols, mid=m ^ rows)
    x = acts(pkg, m, cols, mid=m ^ rows)
    xb = pkg.to_bf16_bits(x)
    x_fed = (xb.astype(np.uint32) << 16).view(np.float32)
    say("q6k gemm bf16", m, rows, cols)
    d_w, d_x = up(torch, raw), up(torch, xb.view(np.int16))
    d_y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
    pkg.qgemm(Q6_K, d_w.data_ptr(), raw.size, d_x.data_ptr(), pkg.BF16, d_y.data_ptr(), m, rows,
              cols, stream(torch))
    torch.cuda.synchronize()
    y = down(d_y)
    assert np.isfinite(y).all()
    toks = sorted({0, 1, m // 2, m - 1})
    ref = orc.forward_linear_batch(Q6_K, raw, x_fed[toks], rows, cols, 8)
    deq = orc.dequantize(Q6_K, raw, rows * cols).reshape(rows, cols)
    err = errlog(f"q6k gemm bf16 {m}x{rows}x{cols}", orc.normalized_error(y[toks], ref, deq,
                                                                          x_fed[toks]),
                 path="gemm_bf16")
    assert err <= 4e-4


def test_q6k_gemm_int8_refused(pkg, torch_dev):
    torch = torch_dev
    raw = weights(pkg, Q6_K, 64, 512)
    d_w = up(torch, raw)
    d_q = torch.zeros(8 * 512 // 32 * 34, dtype=torch.uint8, device="cuda")
    d_y = torch.zeros((8, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(pkg.GpuError) as e:
        pkg.qgemm(Q6_K, d_w.data_ptr(), raw.size, d_q.data_ptr(), 8, d_y.data_ptr(), 8, 64, 512,
                  stream(torch))
    assert e.value.code == pkg.EDTYPE
