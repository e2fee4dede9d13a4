"""Scratch memory of swamp_qgemv_batched and swamp_qgemm (include/swamp_qmm.h,
"Scratch"): split reductions summed in piece order are bit-reproducible,
the per-(device, stream) buffer can be reserved ahead of a graph capture,
a capture without it takes the path without scratch (still within the
contract), and the decompositions that only some shapes reach are checked
against the oracle."""
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K, F32, BF16 = 2, 8, 12, 14, 0, 30
TOL = 1e-3
HIP_STREAM_PER_THREAD = 2  # hipStreamPerThread


@pytest.fixture(scope="module")
def torch_dev(pkg):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    pkg.init()
    return torch


def weights(pkg, dtype, rows, cols, mid):
    return pkg.synth_quantized(dtype, 0x5EED ^ (11 << 32) ^ mid, 0.02, rows, cols)


def acts(pkg, n, cols, mid):
    return pkg.fill_normal(0x5EED ^ 0xA11CE ^ (11 << 32) ^ mid, 1.0, n, cols)


def bf16(pkg, x):
    xb = pkg.to_bf16_bits(x)
    return xb, (xb.astype(np.uint32) << 16).view(np.float32)


def oracle_err(pkg, orc, dtype, raw, rows, cols, y, xs, row_sets=None):
    rb = pkg.row_bytes(dtype, cols)
    worst = 0.0
    for r0, r1 in row_sets or [(0, rows)]:
        sub = raw[r0 * rb:r1 * rb]
        ref = orc.forward_linear_batch(dtype, sub, xs, r1 - r0, cols, 8)
        deq = orc.dequantize(dtype, sub, (r1 - r0) * cols).reshape(r1 - r0, cols)
        worst = max(worst, orc.normalized_error(y[:, r0:r1], ref, deq, xs))
    return worst


def test_workspace_queries(pkg, torch_dev):
    L = pkg.gpu_lib()
    # few tiles: K split into pieces -> scratch
    assert L.swamp_qgemm_workspace(Q4_0, BF16, 64, 512, 4096) > 0
    assert L.swamp_qgemm_workspace(Q4_0, Q8_0, 64, 512, 4096) > 0
    # a full round of tiles on the fused kernel: no split
    assert L.swamp_qgemm_workspace(Q4_0, BF16, 512, 28672, 4096) == 0
    # full rounds plus a last round of half tiles: no split either
    assert L.swamp_qgemm_workspace(Q4_0, BF16, 2048, 28672, 4096) == 0
    # between half a round and one round of full tiles at 2048 tokens, and Q6_K:
    # the dequantize-once route (a bf16 weight chunk)
    assert L.swamp_qgemm_workspace(Q4_0, BF16, 2048, 6144, 4096) >= 6144 * 4096 * 2
    assert L.swamp_qgemm_workspace(Q6_K, BF16, 64, 512, 4096) >= 512 * 4096 * 2
    # small batch: K groups on a short matrix (also with token groups, 40
    # tokens); more than 64 tokens: bf16 x for the GEMM
    assert L.swamp_qgemv_batched_workspace(Q4_K, 16, 4096, 14336, 0) > 0
    assert L.swamp_qgemv_batched_workspace(Q4_0, 40, 4096, 4096, 0) > 0
    assert L.swamp_qgemv_batched_workspace(Q4_0, 80, 4096, 4096, 0) >= 80 * 4096 * 2
    assert L.swamp_qgemv_batched_workspace(Q4_K, 1, 4096, 14336, 0) == 0
    assert L.swamp_workspace_reserve(None, 0) == 0


def test_bench_route_labels_match_library(pkg, torch_dev, monkeypatch):
    """bench.py names the kernels behind each prefill line by the library's
    route rule.  The workspace the library asks for follows the route it
    takes (SWAMP_GEMM_ROUTE forces one, read per call), so on every bench
    shape whose two routes need different scratch, the default's scratch
    names the route, and the label must agree with it."""
    import importlib.util
    import os
    torch = torch_dev
    spec = importlib.util.spec_from_file_location(
        "bench_mod", os.path.join(os.path.dirname(os.path.dirname(__file__)), "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    L = pkg.gpu_lib()
    shapes = [(Q4_0, m, rows, k) for m in (2048, 512) for _, rows, k in bench.PREFILL_SHAPES]
    shapes += [(Q4_K, 4096, rows, k) for _, rows, k in bench.SWEEP_70B]
    # either side of the 1024-token bound (224 tiles: more than half a round)
    shapes += [(Q4_0, 1024, 14336, 4096), (Q4_0, 1000, 14336, 4096)]
    checked = 0
    for dt, m, rows, k in shapes:
        def ws(route=None):
            if route:
                monkeypatch.setenv("SWAMP_GEMM_ROUTE", route)
            else:
                monkeypatch.delenv("SWAMP_GEMM_ROUTE", raising=False)
            return L.swamp_qgemm_workspace(dt, BF16, m, rows, k)
        ws_dq, ws_fused, ws_default = ws("dq"), ws("fused"), ws()
        label = bench.gemm_route(torch, False, m, rows, k, "bf16")
        if ws_dq == ws_fused:
            continue
        assert ws_default in (ws_dq, ws_fused), (dt, m, rows, k)
        assert label.startswith("dequantize-once") == (ws_default == ws_dq), (dt, m, rows, k, label)
        checked += 1
    assert checked >= 6, checked
    # Q6_K always takes the dequantize-once route
    assert bench.gemm_route(torch, True, 64, 512, 4096, "bf16").startswith("dequantize-once")


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
def test_gemm_int8_split_repeat_bitwise(pkg, orc, torch_dev, errlog, dtype):
    """The int8 GEMM's K pieces are summed in piece order: repeated calls,
    with other shapes in between, give identical bits."""
    torch = torch_dev
    s = torch.cuda.current_stream().cuda_stream
    cases = [(64, 512, 4096), (8, 1000, 14336), (300, 256, 2048)]
    first = {}
    for rep in range(3):
        for m, rows, cols in cases:
            raw = weights(pkg, dtype, rows, cols, mid=m ^ rows)
            x = acts(pkg, m, cols, mid=m ^ rows)
            print(f"[gpu case] int8 repeat {dtype} {m}x{rows}x{cols} rep {rep}", flush=True)
            d_w, d_x = torch.from_numpy(raw).cuda(), torch.from_numpy(x).cuda()
            d_q = torch.empty(m * cols // 32 * 34, dtype=torch.uint8, device="cuda")
            pkg.quantize_q8_0(d_x.data_ptr(), F32, d_q.data_ptr(), m * cols, s)
            d_y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
            pkg.qgemm(dtype, d_w.data_ptr(), raw.size, d_q.data_ptr(), Q8_0, d_y.data_ptr(), m,
                      rows, cols, s)
            torch.cuda.synchronize()
            y = d_y.cpu().numpy()
            key = (m, rows, cols)
            if rep == 0:
                first[key] = y
                xq = d_q.cpu().numpy()
                x_fed = orc.dequantize(Q8_0, xq, m * cols).reshape(m, cols)
                toks = sorted({0, m // 2, m - 1})
                err = oracle_err(pkg, orc, dtype, raw, rows, cols, y[toks], x_fed[toks])
                errlog(f"int8 split {dtype} {m}x{rows}x{cols}", err, path="gemm_i8")
                assert err <= 1e-5
            else:
                assert np.array_equal(y.view(np.uint32), first[key].view(np.uint32)), (key, rep)


@pytest.mark.parametrize("x_type,m,rows,cols", [(BF16, 512, 6144, 4096), (BF16, 2048, 4096, 14336),
                                                 (Q8_0, 512, 4096, 14336), (BF16, 40, 3000, 4096)])
def test_split_sum_vector_and_scalar_bitwise(pkg, torch_dev, x_type, m, rows, cols):
    """The K pieces' sum runs 4 elements per thread when y is 16-byte aligned
    (and one per thread otherwise, here y one float past an aligned address):
    both take the same additions in piece order, so y is the same bits."""
    torch = torch_dev
    s = torch.cuda.current_stream().cuda_stream
    raw = weights(pkg, Q4_0, rows, cols, mid=m ^ rows)
    x = acts(pkg, m, cols, mid=m ^ rows)
    print(f"[gpu case] split sum {x_type} {m}x{rows}x{cols}", flush=True)
    d_w = torch.from_numpy(raw).cuda()
    if x_type == BF16:
        d_x = torch.from_numpy(pkg.to_bf16_bits(x).view(np.int16)).cuda()
    else:
        d_f = torch.from_numpy(x).cuda()
        d_x = torch.empty(m * cols // 32 * 34, dtype=torch.uint8, device="cuda")
        pkg.quantize_q8_0(d_f.data_ptr(), F32, d_x.data_ptr(), m * cols, s)
    buf = torch.full((m * rows + 4,), float("nan"), dtype=torch.float32, device="cuda")
    assert buf.data_ptr() % 16 == 0
    ys = []
    for off in (0, 1):
        pkg.qgemm(Q4_0, d_w.data_ptr(), raw.size, d_x.data_ptr(), x_type,
                  buf.data_ptr() + 4 * off, m, rows, cols, s)
        torch.cuda.synchronize()
        ys.append(buf.cpu().numpy()[off:off + m * rows].copy())
    assert np.all(np.isfinite(ys[0]))
    assert np.array_equal(ys[0].view(np.uint32), ys[1].view(np.uint32))


@pytest.mark.parametrize("dtype", [Q4_0, Q8_0, Q4_K])
@pytest.mark.parametrize("m,rows,cols", [(24, 33024, 1024), (64, 128256, 4096)])
def test_gemm_small_m_single_piece(pkg, orc, torch_dev, errlog, dtype, m, rows, cols):
    """At most 64 tokens with more than half a round of 64-token tiles: the
    single-piece form of the small-M GEMM (no K split), which the 64-token
    sweep times on the lm_head."""
    torch = torch_dev
    if dtype == Q4_K and cols % 256:
        pytest.skip("Q4_K rows are whole 256-blocks")
    s = torch.cuda.current_stream().cuda_stream
    assert pkg.gpu_lib().swamp_qgemm_workspace(dtype, BF16, m, rows, cols) == 0
    raw = weights(pkg, dtype, rows, cols, mid=rows ^ m)
    xb, x_fed = bf16(pkg, acts(pkg, m, cols, mid=rows ^ m))
    print(f"[gpu case] gemm small m single piece {dtype} {m}x{rows}x{cols}", flush=True)
    d_w, d_x = torch.from_numpy(raw).cuda(), torch.from_numpy(xb.view(np.int16)).cuda()
    d_y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
    pkg.qgemm(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), BF16, d_y.data_ptr(), m, rows, cols,
              s)
    torch.cuda.synchronize()
    y = d_y.cpu().numpy()
    assert np.isfinite(y).all()
    toks = sorted({0, 1, m // 2, m - 1})
    err = oracle_err(pkg, orc, dtype, raw, rows, cols, y[toks], x_fed[toks],
                     [(0, 512), (rows // 2 - 256, rows // 2 + 256), (rows - 512, rows)])
    errlog(f"gemm small-m single piece {dtype} {m}x{rows}x{cols}", err, path="gemm_bf16")
    assert err <= 4e-4


def _calls(pkg, torch, mid):
    """Calls that take scratch: small batch with K groups (16 tokens, and
    40 in token groups), small batch of 80 tokens (bf16 x + GEMM pieces),
    GEMM split into pieces."""
    out = []
    for kind, dtype, n, rows, cols in [("batched", Q4_K, 16, 4096, 14336),
                                       ("batched", Q4_K, 40, 1024, 4096),
                                       ("batched", Q4_0, 80, 1024, 4096),
                                       ("gemm", Q8_0, 64, 512, 4096)]:
        raw = weights(pkg, dtype, rows, cols, mid=mid ^ rows)
        x = acts(pkg, n, cols, mid=mid ^ rows)
        if kind == "gemm":
            xb, x_fed = bf16(pkg, x)
            d_x = torch.from_numpy(xb.view(np.int16)).cuda()
        else:
            x_fed = x
            d_x = torch.from_numpy(x).cuda()
        out.append(dict(kind=kind, dtype=dtype, n=n, rows=rows, cols=cols, raw=raw,
                        d_w=torch.from_numpy(raw).cuda(), d_x=d_x, x_fed=x_fed,
                        d_y=torch.full((n, rows), float("nan"), dtype=torch.float32,
                                       device="cuda")))
    return out


def _run(pkg, c, s):
    if c["kind"] == "batched":
        pkg.qgemv_batched(c["dtype"], c["d_w"].data_ptr(), c["raw"].size, c["d_x"].data_ptr(),
                          c["d_y"].data_ptr(), c["n"], c["rows"], c["cols"], False, s)
    else:
        pkg.qgemm(c["dtype"], c["d_w"].data_ptr(), c["raw"].size, c["d_x"].data_ptr(), BF16,
                  c["d_y"].data_ptr(), c["n"], c["rows"], c["cols"], s)


def _need(pkg, c):
    L = pkg.gpu_lib()
    if c["kind"] == "batched":
        return L.swamp_qgemv_batched_workspace(c["dtype"], c["n"], c["rows"], c["cols"], 0)
    return L.swamp_qgemm_workspace(c["dtype"], BF16, c["n"], c["rows"], c["cols"])


def test_graph_capture_with_reserved_scratch(pkg, torch_dev):
    """Scratch reserved on a stream before capture: the captured calls use
    it, and every replay (with eager work and synchronisations in between)
    gives the eager result bit for bit."""
    torch = torch_dev
    cs = torch.cuda.Stream()  # default priority
    calls = _calls(pkg, torch, mid=1)
    need = max(_need(pkg, c) for c in calls)
    assert need > 0
    print("[gpu case] graph capture with reserved scratch", flush=True)
    with torch.cuda.stream(cs):
        pkg.workspace_reserve(cs.cuda_stream, need)
        for c in calls:
            _run(pkg, c, cs.cuda_stream)
    torch.cuda.synchronize()
    eager = [c["d_y"].cpu().numpy().copy() for c in calls]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        for c in calls:
            _run(pkg, c, cs.cuda_stream)
    for rep in range(3):
        for c in calls:
            c["d_y"].fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for c, e in zip(calls, eager):
            assert np.array_equal(c["d_y"].cpu().numpy().view(np.uint32), e.view(np.uint32)), rep


def test_graph_keeps_scratch_after_larger_eager_call(pkg, torch_dev):
    """Reserve, capture, then an eager call on the same stream that needs a
    larger buffer: the stream's buffer is replaced, but the one the graph
    holds stays allocated, and every replay still gives the eager bits."""
    torch = torch_dev
    cs = torch.cuda.Stream()
    calls = _calls(pkg, torch, mid=3)
    need = max(_need(pkg, c) for c in calls)
    print("[gpu case] graph replay after a larger eager call", flush=True)
    with torch.cuda.stream(cs):
        pkg.workspace_reserve(cs.cuda_stream, need)
        for c in calls:
            _run(pkg, c, cs.cuda_stream)
    torch.cuda.synchronize()
    eager = [c["d_y"].cpu().numpy().copy() for c in calls]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        for c in calls:
            _run(pkg, c, cs.cuda_stream)
    # a Q6_K prefill: the dequantize-once route, whose bf16 weight chunk is
    # far larger than the reservation
    rows, cols, n = 1024, 4096, 64
    big = pkg.gpu_lib().swamp_qgemm_workspace(Q6_K, BF16, n, rows, cols)
    assert big > need
    raw = weights(pkg, Q6_K, rows, cols, mid=7)
    d_w = torch.from_numpy(raw).cuda()
    d_x = torch.from_numpy(bf16(pkg, acts(pkg, n, cols, mid=7))[0].view(np.int16)).cuda()
    d_y = torch.empty((n, rows), dtype=torch.float32, device="cuda")
    for rep in range(3):
        with torch.cuda.stream(cs):
            pkg.qgemm(Q6_K, d_w.data_ptr(), raw.size, d_x.data_ptr(), BF16, d_y.data_ptr(), n,
                      rows, cols, cs.cuda_stream)
        torch.cuda.synchronize()
        for c in calls:
            c["d_y"].fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for c, e in zip(calls, eager):
            assert np.array_equal(c["d_y"].cpu().numpy().view(np.uint32), e.view(np.uint32)), rep


def test_graph_capture_without_scratch(pkg, orc, torch_dev, errlog):
    """A fresh stream captured without a reservation allocates nothing: the
    calls take the path without scratch (K pieces and K groups added with
    float atomics into y cleared by a kernel; more than 64 tokens in passes
    of 64), which stays within the contract on every replay."""
    torch = torch_dev
    cs = torch.cuda.Stream()
    calls = _calls(pkg, torch, mid=2)
    print("[gpu case] graph capture without scratch", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        for c in calls:
            _run(pkg, c, cs.cuda_stream)
    for rep in range(3):
        for c in calls:
            c["d_y"].fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for c in calls:
            y = c["d_y"].cpu().numpy()
            assert np.isfinite(y).all()
            toks = sorted({0, c["n"] // 2, c["n"] - 1})
            err = oracle_err(pkg, orc, c["dtype"], c["raw"], c["rows"], c["cols"], y[toks],
                             c["x_fed"][toks])
            if rep == 0:
                errlog(f"no-scratch {c['kind']} {c['dtype']} n={c['n']}", err,
                       path="no_scratch")
            assert err <= 4e-4, (c["kind"], c["dtype"], rep)


def test_per_thread_default_stream(pkg, torch_dev):
    """hipStreamPerThread is one handle for several streams: two host threads
    calling on it at once each get their own scratch, so both give the bits
    of the same calls run alone."""
    torch = torch_dev
    calls = [_calls(pkg, torch, mid=3 + t) for t in range(2)]
    print("[gpu case] hipStreamPerThread from two host threads", flush=True)
    ref = []
    for cl in calls:
        for c in cl:
            _run(pkg, c, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        ref.append([c["d_y"].cpu().numpy().copy() for c in cl])
        for c in cl:
            c["d_y"].fill_(float("nan"))
    torch.cuda.synchronize()
    errors = []

    def work(cl):
        try:
            for _ in range(4):
                for c in cl:
                    _run(pkg, c, HIP_STREAM_PER_THREAD)
            if pkg.gpu_lib().gpu_stream_synchronize(HIP_STREAM_PER_THREAD) != 0:
                errors.append("sync")
        except Exception as e:  # reported below
            errors.append(repr(e))

    th = [threading.Thread(target=work, args=(cl,)) for cl in calls]
    for t in th:
        t.start()
    for t in th:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for cl, r in zip(calls, ref):
        for c, e in zip(cl, r):
            assert np.array_equal(c["d_y"].cpu().numpy().view(np.uint32), e.view(np.uint32))


@pytest.mark.parametrize("accumulate", [False, True])
def test_batched_large_activation_within_fp16_range(pkg, orc, torch_dev, errlog, accumulate):
    """The 2..64-token passes round x to fp16: an activation of 6e4 (inside
    fp16 range, documented limit |x| < 65504) still gives results within
    the contract, also on the accumulating form."""
    torch = torch_dev
    s = torch.cuda.current_stream().cuda_stream
    n, rows, cols = 8, 1024, 4096
    raw = weights(pkg, Q4_K, rows, cols, mid=77)
    x = acts(pkg, n, cols, mid=77)
    x[3, 100] = 6.0e4
    x[5, 4000] = -6.0e4
    base = np.zeros((n, rows), np.float32)
    d_w, d_x = torch.from_numpy(raw).cuda(), torch.from_numpy(x).cuda()
    d_y = torch.from_numpy(base.copy()).cuda()
    pkg.qgemv_batched(Q4_K, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), n, rows,
                      cols, accumulate, s)
    torch.cuda.synchronize()
    y = d_y.cpu().numpy()
    assert np.isfinite(y).all()
    err = oracle_err(pkg, orc, Q4_K, raw, rows, cols, y, x)
    errlog(f"batched |x| = 6e4 accumulate={accumulate}", err, path="batched_f16")
    assert err <= TOL
