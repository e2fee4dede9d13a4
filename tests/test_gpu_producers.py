"""GPU parity of the activation producers (swamp_rmsnorm_rows, swamp_swiglu)
against the oracle's rmsnorm and silu + mul_in_place (swamp-engine/src/
ops.rs:188-214), and of their use in front of the small batch and the prefill
GEMM against forward_linear per token on the fed activations.

Gates:
  * fp32 output: |out - ref| <= 3e-5 |ref| elementwise for RMSNorm (the sum of
    squares runs in another order; every element of a row shares the relative
    error of inv_rms) and <= 2e-6 |ref| + 1e-30 for SwiGLU (exp2 and reciprocal
    within about 1 ulp each against the C library's expf);
  * bf16 output: bit-equal to the round-to-nearest-even of the same call's
    fp32 output;
  * matmuls fed by a producer: max_r |y - y_ref| / (||W_r|| ||x_fed||) <= 1e-3
    with x_fed the values the producer wrote."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_0, Q4_K = 2, 12
F32, BF16 = 0, 30
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


def stream(torch):
    return torch.cuda.current_stream().cuda_stream


def say(*a):
    print("[gpu case]", *a, flush=True)


def bf16_bits_to_f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def run_rmsnorm(pkg, torch, x, w, eps, out_type):
    n_tok, cols = x.shape
    dx, dw = up(torch, x), up(torch, w)
    if out_type == F32:
        out = torch.empty((n_tok, cols), dtype=torch.float32, device="cuda")
    else:
        out = torch.empty((n_tok, cols), dtype=torch.int16, device="cuda")
    pkg.rmsnorm_rows(dx.data_ptr(), dw.data_ptr(), eps, out.data_ptr(), out_type, n_tok, cols,
                     stream(torch))
    torch.cuda.synchronize()
    res = out.cpu().numpy()
    return res if out_type == F32 else res.view(np.uint16)


def run_swiglu(pkg, torch, g, u, out_type):
    n = g.size
    dg, du = up(torch, g), up(torch, u)
    out = torch.empty(n, dtype=torch.float32 if out_type == F32 else torch.int16, device="cuda")
    pkg.swiglu(dg.data_ptr(), du.data_ptr(), out.data_ptr(), out_type, n, stream(torch))
    torch.cuda.synchronize()
    res = out.cpu().numpy()
    return res if out_type == F32 else res.view(np.uint16)


@pytest.mark.parametrize("n_tok,cols", [(1, 4096), (5, 14336), (16, 8192), (3, 100), (2, 8)])
def test_rmsnorm_rows(pkg, orc, torch_dev, n_tok, cols):
    say("rmsnorm_rows", n_tok, cols)
    x = pkg.fill_normal(SEED ^ 0x51, 1.0, n_tok, cols)
    x[0, :4] = [30.0, -30.0, 1e-3, 0.0]  # a few large and tiny entries
    w = pkg.fill_normal(SEED ^ 0x52, 0.5, 1, cols)[0] + 1.0
    eps = 1e-5
    out = run_rmsnorm(pkg, torch_dev, x, w, eps, F32)
    ref = np.stack([orc.rmsnorm(x[t], w, eps) for t in range(n_tok)])
    assert np.all(np.abs(out - ref) <= 3e-5 * np.abs(ref)), np.max(np.abs(out - ref) / (np.abs(ref) + 1e-30))
    bits = run_rmsnorm(pkg, torch_dev, x, w, eps, BF16)
    assert np.array_equal(bits, pkg.to_bf16_bits(out).reshape(n_tok, cols))


def test_rmsnorm_rows_zero_row(pkg, orc, torch_dev):
    """An all-zero row gives inv = 1/sqrt(eps) and zeros out (no NaN)."""
    x = np.zeros((2, 256), dtype=np.float32)
    x[1] = 1.0
    w = np.ones(256, dtype=np.float32)
    out = run_rmsnorm(pkg, torch_dev, x, w, 1e-6, F32)
    assert np.all(out[0] == 0.0)
    assert np.allclose(out[1], orc.rmsnorm(x[1], w, 1e-6), rtol=3e-6, atol=0)


@pytest.mark.parametrize("n", [4, 4096, 14336 * 5, 1 << 20])
def test_swiglu(pkg, orc, torch_dev, n):
    say("swiglu", n)
    g = pkg.fill_normal(SEED ^ 0x61, 3.0, 1, n)[0]
    u = pkg.fill_normal(SEED ^ 0x62, 1.0, 1, n)[0]
    g[:4] = [-100.0, 100.0, 0.0, -0.5]
    out = run_swiglu(pkg, torch_dev, g, u, F32)
    ref = orc.silu(g) * u
    assert np.all(np.abs(out - ref) <= 2e-6 * np.abs(ref) + 1e-30), np.max(np.abs(out - ref))
    bits = run_swiglu(pkg, torch_dev, g, u, BF16)
    assert np.array_equal(bits, pkg.to_bf16_bits(out).reshape(-1))


@pytest.mark.parametrize("dtype", [Q4_0, Q4_K])
def test_rmsnorm_then_gemm(pkg, orc, torch_dev, dtype):
    """RMSNorm rows written as bf16 feed the prefill GEMM directly."""
    torch = torch_dev
    m, rows, cols = 96, 384, 4096
    say("rmsnorm -> gemm", dtype, m, rows, cols)
    x = pkg.fill_normal(SEED ^ 0x71, 1.0, m, cols)
    w = pkg.fill_normal(SEED ^ 0x72, 0.5, 1, cols)[0] + 1.0
    dx, dw = up(torch, x), up(torch, w)
    xb = torch.empty((m, cols), dtype=torch.int16, device="cuda")
    pkg.rmsnorm_rows(dx.data_ptr(), dw.data_ptr(), 1e-5, xb.data_ptr(), BF16, m, cols,
                     stream(torch))
    raw = pkg.synth_quantized(dtype, SEED ^ 0x73, 0.02, rows, cols)
    dwt = up(torch, raw)
    y = torch.empty((m, rows), dtype=torch.float32, device="cuda")
    pkg.qgemm(dtype, dwt.data_ptr(), raw.size, xb.data_ptr(), BF16, y.data_ptr(), m, rows, cols,
              stream(torch))
    torch.cuda.synchronize()
    fed = bf16_bits_to_f32(xb.cpu().numpy().view(np.uint16))
    yh = y.cpu().numpy()
    deq = orc.dequantize(dtype, raw, rows * cols).reshape(rows, cols)
    worst = 0.0
    for t in range(0, m, 7):
        ref = orc.forward_linear(dtype, raw, fed[t], rows, cols, 8)
        worst = max(worst, orc.normalized_error(yh[t], ref, deq, fed[t]))
    assert worst <= TOL, worst


def test_swiglu_then_batched(pkg, orc, torch_dev):
    """SwiGLU rows written as fp32 feed the small batch (the down projection)."""
    torch = torch_dev
    n_tok, rows, cols = 8, 512, 14336
    say("swiglu -> batched", n_tok, rows, cols)
    g = pkg.fill_normal(SEED ^ 0x81, 2.0, n_tok, cols)
    u = pkg.fill_normal(SEED ^ 0x82, 1.0, n_tok, cols)
    dg, du = up(torch, g), up(torch, u)
    h = torch.empty((n_tok, cols), dtype=torch.float32, device="cuda")
    pkg.swiglu(dg.data_ptr(), du.data_ptr(), h.data_ptr(), F32, n_tok * cols, stream(torch))
    raw = pkg.synth_quantized(Q4_K, SEED ^ 0x83, 0.02, rows, cols)
    dwt = up(torch, raw)
    y = torch.empty((n_tok, rows), dtype=torch.float32, device="cuda")
    pkg.qgemv_batched(Q4_K, dwt.data_ptr(), raw.size, h.data_ptr(), y.data_ptr(), n_tok, rows,
                      cols, 0, stream(torch))
    torch.cuda.synchronize()
    fed = h.cpu().numpy()
    yh = y.cpu().numpy()
    deq = orc.dequantize(Q4_K, raw, rows * cols).reshape(rows, cols)
    worst = 0.0
    for t in range(n_tok):
        ref = orc.forward_linear(Q4_K, raw, fed[t], rows, cols, 8)
        worst = max(worst, orc.normalized_error(yh[t], ref, deq, fed[t]))
    assert worst <= TOL, worst
