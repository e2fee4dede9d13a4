"""GPU parity of the fused-prologue GEMVs against the oracle's composition of
the engine's steps: rmsnorm (swamp-engine/src/ops.rs:188-201) then
forward_linear per matrix (linear.rs:14-90, 96-170), and silu + mul_in_place
+ forward_linear + add_in_place (ops.rs:203-220, executor.rs:501-506).
Gate: max_r |y - y_ref| / (||W_r|| ||x_fed||) <= 1e-3 with x_fed the oracle's
normalized / gated vector.  Also the n_cols == 0 contract (y = 0)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
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
    return pkg.synth_quantized(dtype, SEED ^ (11 << 32) ^ mid, 0.02, rows, cols)


def acts(pkg, n, cols, mid=0):
    return pkg.fill_normal(SEED ^ 0xF00 ^ mid, 1.0, n, cols)


def _err(pkg, orc, dt, raw, x_fed, y, rows, cols, sel=None):
    rb = pkg.row_bytes(dt, cols)
    worst = 0.0
    for r0, r1 in sel or [(0, rows)]:
        sub = raw[r0 * rb:r1 * rb]
        ref = orc.forward_linear(dt, sub, x_fed, r1 - r0, cols, 8)
        deq = orc.dequantize(dt, sub, (r1 - r0) * cols).reshape(r1 - r0, cols)
        worst = max(worst, orc.normalized_error(y[r0:r1], ref, deq, x_fed))
    return worst


# Llama-3 8B: QKV (Q4_K_M keeps attn_v in Q6_K), gate+up, 70B QKV, logits
RMS_CASES = [
    ("8b qkv q4_0", 4096, [(Q4_0, 4096), (Q4_0, 1024), (Q4_0, 1024)]),
    ("8b qkv q4_k_m", 4096, [(Q4_K, 4096), (Q4_K, 1024), (Q6_K, 1024)]),
    ("8b gate_up q4_k", 4096, [(Q4_K, 14336), (Q4_K, 14336)]),
    ("8b gate_up q8_0", 4096, [(Q8_0, 14336), (Q8_0, 14336)]),
    ("70b qkv q4_k", 8192, [(Q4_K, 8192), (Q4_K, 1024), (Q4_K, 1024)]),
    ("small odd", 320, [(Q4_0, 77), (Q8_0, 5)]),
]


@pytest.mark.parametrize("name,cols,spec", RMS_CASES, ids=[c[0] for c in RMS_CASES])
def test_rmsnorm_gemv_parity(pkg, orc, torch_dev, name, cols, spec):
    torch = torch_dev
    raws = [weights(pkg, dt, r, cols, mid=i) for i, (dt, r) in enumerate(spec)]
    x, wn = acts(pkg, 2, cols, mid=cols)
    x = (x * 7.0).astype(np.float32)  # the residual stream is not unit-scale
    wn = (1.0 + 0.2 * wn).astype(np.float32)
    eps = 1e-5
    d_ws = [up(torch, r) for r in raws]
    d_ys = [torch.full((r,), float("nan"), dtype=torch.float32, device="cuda") for _, r in spec]
    d_x, d_wn = up(torch, x), up(torch, wn)
    say("rmsnorm gemv", name)
    pkg.qgemv_rmsnorm([dt for dt, _ in spec], [t.data_ptr() for t in d_ws], [r.size for r in raws],
                      [r for _, r in spec], d_x.data_ptr(), d_wn.data_ptr(), eps,
                      [t.data_ptr() for t in d_ys], cols, stream(torch))
    torch.cuda.synchronize()
    x_norm = orc.rmsnorm(x, wn, eps)
    for (dt, r), raw, d_y in zip(spec, raws, d_ys):
        y = down(d_y)
        assert np.all(np.isfinite(y))
        e = _err(pkg, orc, dt, raw, x_norm, y, r, cols)
        assert e <= TOL, (dt, r, e)


def test_rmsnorm_gemv_logits_and_scale(pkg, orc, torch_dev):
    """The logits (Q6_K lm_head, 128256 x 4096) after the final norm, on
    three row ranges; with eps = 0 the fused result is unchanged when x is
    scaled by 2^20 (the normalization is exact under powers of two)."""
    torch = torch_dev
    rows, cols = 128256, 4096
    raw = weights(pkg, Q6_K, rows, cols, mid=77)
    x, wn = acts(pkg, 2, cols, mid=77)
    wn = (1.0 + 0.2 * wn).astype(np.float32)
    d_w, d_wn = up(torch, raw), up(torch, wn)
    outs = []
    say("rmsnorm logits")
    for xv in (x, x * np.float32(2.0 ** 20)):
        d_x = up(torch, xv.astype(np.float32))
        d_y = torch.empty(rows, dtype=torch.float32, device="cuda")
        pkg.qgemv_rmsnorm([Q6_K], [d_w.data_ptr()], [raw.size], [rows], d_x.data_ptr(),
                          d_wn.data_ptr(), 0.0, [d_y.data_ptr()], cols, stream(torch))
        outs.append(down(d_y))
    torch.cuda.synchronize()
    assert np.array_equal(outs[0], outs[1])
    x_norm = orc.rmsnorm(x, wn, 0.0)
    e = _err(pkg, orc, Q6_K, raw, x_norm, outs[0], rows, cols,
             sel=[(0, 1024), (rows // 2, rows // 2 + 512), (rows - 1024, rows)])
    assert e <= TOL, e


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K, Q6_K])
@pytest.mark.parametrize("rows,cols", [(4096, 14336), (8192, 28672), (300, 1024)])
@pytest.mark.parametrize("accumulate", [False, True])
def test_swiglu_down_parity(pkg, orc, torch_dev, dtype, rows, cols, accumulate):
    torch = torch_dev
    raw = weights(pkg, dtype, rows, cols, mid=rows ^ dtype)
    g, u = acts(pkg, 2, cols, mid=cols ^ dtype)
    g = (g * 3.0).astype(np.float32)
    resid = acts(pkg, 1, rows, mid=rows)[0]
    d_w, d_g, d_u = up(torch, raw), up(torch, g), up(torch, u)
    d_y = up(torch, resid) if accumulate else torch.full((rows,), float("nan"),
                                                         dtype=torch.float32, device="cuda")
    say("swiglu down", dtype, rows, cols, accumulate)
    pkg.qgemv_swiglu(dtype, d_w.data_ptr(), raw.size, d_g.data_ptr(), d_u.data_ptr(),
                     d_y.data_ptr(), rows, cols, accumulate, stream(torch))
    torch.cuda.synchronize()
    y = down(d_y)
    h = orc.mul_in_place(orc.silu(g), u)
    if accumulate:
        ref_full = orc.add_in_place(resid, orc.forward_linear(dtype, raw, h, rows, cols, 8))
        deq = orc.dequantize(dtype, raw, rows * cols).reshape(rows, cols)
        # the residual add rounds once more: normalized by ||W_r|| ||h||
        assert orc.normalized_error(y, ref_full, deq, h) <= TOL
    else:
        assert np.all(np.isfinite(y))
        assert _err(pkg, orc, dtype, raw, h, y, rows, cols) <= TOL


def test_fused_equal_unfused_bitwise_on_plain_path(pkg, orc, torch_dev):
    """Feeding the GEMV the oracle's x_norm vs the fused RMSNorm: both within
    the gate, and the plain GEMV of the fused kernel's own input matches the
    fused result to fp16-rounding level (2^-11 relative)."""
    torch = torch_dev
    rows, cols = 2048, 4096
    raw = weights(pkg, Q4_K, rows, cols, mid=5)
    x, wn = acts(pkg, 2, cols, mid=5)
    wn = (1.0 + 0.2 * wn).astype(np.float32)
    x_norm = orc.rmsnorm(x, wn, 1e-5)
    d_w, d_x, d_wn, d_xn = up(torch, raw), up(torch, x), up(torch, wn), up(torch, x_norm)
    y_f = torch.empty(rows, dtype=torch.float32, device="cuda")
    y_p = torch.empty(rows, dtype=torch.float32, device="cuda")
    pkg.qgemv_rmsnorm([Q4_K], [d_w.data_ptr()], [raw.size], [rows], d_x.data_ptr(),
                      d_wn.data_ptr(), 1e-5, [y_f.data_ptr()], cols, stream(torch))
    pkg.qgemv(Q4_K, d_w.data_ptr(), raw.size, d_xn.data_ptr(), y_p.data_ptr(), rows, cols,
              stream(torch))
    torch.cuda.synchronize()
    deq = orc.dequantize(Q4_K, raw, rows * cols).reshape(rows, cols)
    assert orc.normalized_error(down(y_f), down(y_p), deq, x_norm) <= 2e-4


def test_zero_columns_give_zero(pkg, torch_dev):
    """A sum over no columns is 0 (forward_linear with nc = 0 writes 0): the
    entry points fill y without reading W or x."""
    torch = torch_dev
    s = stream(torch)
    d_w = torch.zeros(64, dtype=torch.uint8, device="cuda")
    d_x = torch.zeros(4, dtype=torch.float32, device="cuda")
    for dt in (Q4_0, Q8_0, Q4_K, Q6_K):
        y = torch.full((37,), float("nan"), dtype=torch.float32, device="cuda")
        pkg.qgemv(dt, d_w.data_ptr(), 0, d_x.data_ptr(), y.data_ptr(), 37, 0, s)
        yb = torch.full((3, 37), float("nan"), dtype=torch.float32, device="cuda")
        pkg.qgemv_batched(dt, d_w.data_ptr(), 0, d_x.data_ptr(), yb.data_ptr(), 3, 37, 0,
                          False, s)
        torch.cuda.synchronize()
        assert not y.isnan().any() and (y == 0).all(), dt
        assert (yb == 0).all(), dt
    ym = torch.full((5, 9), float("nan"), dtype=torch.float32, device="cuda")
    pkg.qgemm(Q4_0, d_w.data_ptr(), 0, d_x.data_ptr(), pkg.BF16, ym.data_ptr(), 5, 9, 0, s)
    torch.cuda.synchronize()
    assert (ym == 0).all()
