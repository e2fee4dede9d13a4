"""swamp_qgemv_batched_noalloc (include/swamp_qmm.h): the allocation-free
variant of swamp_qgemv_batched, with its scratch in a fixed per-GPU device
array.  Through the C ABI, each call's output is compared bit for bit with
swamp_qgemv_batched on the same inputs (both sum split reductions in a fixed
order), on two calls in a row, the second with a smaller input, and with
the oracle; on a fresh stream the calls leave the device's default memory
pool (where the library's per-stream scratch comes from) untouched, while
the same calls through swamp_qgemv_batched take from it; a call whose
scratch exceeds the array is refused before anything is launched."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K = 2, 8, 12
EWORKSPACE = -6
MAX_SCRATCH = 32 << 20


@pytest.fixture(scope="module")
def torch_dev(pkg):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    pkg.init()
    return torch


def _case(pkg, torch, dtype, n_tok, rows, cols, mid):
    raw = pkg.synth_quantized(dtype, 0x5EED ^ (13 << 32) ^ mid, 0.02, rows, cols)
    xs = pkg.fill_normal(0x5EED ^ 0xA11CE ^ (13 << 32) ^ mid, 1.0, n_tok, cols)
    return raw, xs, torch.from_numpy(raw).cuda(), torch.from_numpy(xs).cuda()


def test_noalloc_matches_batched_two_calls(pkg, orc, torch_dev, errlog):
    torch = torch_dev
    L = pkg.gpu_lib()
    s = torch.cuda.current_stream().cuda_stream
    # first call: 80 tokens (bf16 x and K pieces in scratch); second, a
    # smaller input: 8 tokens on a short matrix (K groups in scratch)
    cases = [(Q4_0, 80, 4096, 4096, 1, False), (Q4_K, 8, 1024, 14336, 2, False),
             (Q8_0, 16, 4096, 4096, 3, True)]
    for dtype, n_tok, rows, cols, mid, acc in cases:
        need = L.swamp_qgemv_batched_workspace(dtype, n_tok, rows, cols, int(acc))
        assert 0 < need <= MAX_SCRATCH, need
        raw, xs, d_w, d_x = _case(pkg, torch, dtype, n_tok, rows, cols, mid)
        base = np.random.default_rng(mid).standard_normal((n_tok, rows)).astype(np.float32)
        print(f"[gpu case] noalloc {dtype} n_tok {n_tok} {rows}x{cols} acc {acc}", flush=True)
        outs = []
        for fn in (L.swamp_qgemv_batched_noalloc, L.swamp_qgemv_batched):
            d_y = torch.from_numpy(base.copy()).cuda()
            rc = fn(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), n_tok, rows,
                    cols, int(acc), s)
            assert rc == 0, rc
            torch.cuda.synchronize()
            outs.append(d_y.cpu().numpy())
        assert np.isfinite(outs[0]).all()
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
        ref = base.copy() if acc else np.zeros_like(base)
        ref += orc.forward_linear_batch(dtype, raw, xs, rows, cols, 8)
        deq = orc.dequantize(dtype, raw, rows * cols).reshape(rows, cols)
        err = errlog(f"noalloc {dtype} n_tok={n_tok} {rows}x{cols} acc={acc}",
                     orc.normalized_error(outs[0], ref, deq, xs), path="noalloc")
        assert err <= 1e-3


HIP_MEMPOOL_USED_MEM_CURRENT = 7  # hipMemPoolAttrUsedMemCurrent


def _pool_used(torch):
    """Bytes in use from the current device's default memory pool (the pool
    hipMallocAsync draws from), through the HIP runtime torch has loaded."""
    hip = ctypes.CDLL("libamdhip64.so.7")
    dev = torch.cuda.current_device()
    pool = ctypes.c_void_p()
    assert hip.hipDeviceGetDefaultMemPool(ctypes.byref(pool), dev) == 0
    used = ctypes.c_uint64()
    assert hip.hipMemPoolGetAttribute(pool, HIP_MEMPOOL_USED_MEM_CURRENT, ctypes.byref(used)) == 0
    return used.value


def test_noalloc_allocates_nothing(pkg, torch_dev):
    """On a stream the library has never seen, swamp_qgemv_batched would
    allocate its scratch from the default pool (the positive control below);
    swamp_qgemv_batched_noalloc with the same scratch-taking shape must not."""
    torch = torch_dev
    L = pkg.gpu_lib()
    dtype, n_tok, rows, cols = Q4_K, 16, 4096, 14336  # K groups: partial sums in scratch
    assert L.swamp_qgemv_batched_workspace(dtype, n_tok, rows, cols, 0) > 0
    raw, xs, d_w, d_x = _case(pkg, torch, dtype, n_tok, rows, cols, 5)
    d_y = torch.empty((n_tok, rows), dtype=torch.float32, device="cuda")
    print("[gpu case] noalloc leaves the default memory pool untouched", flush=True)
    for fn, allocates in ((L.swamp_qgemv_batched_noalloc, False), (L.swamp_qgemv_batched, True)):
        cs = torch.cuda.Stream()  # a stream without a library buffer
        torch.cuda.synchronize()
        before = _pool_used(torch)
        for _ in range(2):
            assert fn(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(), d_y.data_ptr(), n_tok, rows,
                      cols, 0, cs.cuda_stream) == 0
        torch.cuda.synchronize()
        after = _pool_used(torch)
        if allocates:
            assert after > before, (before, after)
        else:
            assert after == before, (before, after)


def test_noalloc_rejects_oversized_scratch(pkg, torch_dev):
    torch = torch_dev
    L = pkg.gpu_lib()
    s = torch.cuda.current_stream().cuda_stream
    # 256 tokens, 32 tiles of 256 rows, long K: full tiles in 8 K pieces (67 MB)
    dtype, n_tok, rows, cols = Q4_0, 256, 8192, 32768
    need = L.swamp_qgemv_batched_workspace(dtype, n_tok, rows, cols, 0)
    assert need > MAX_SCRATCH, need
    raw, xs, d_w, d_x = _case(pkg, torch, dtype, n_tok, rows, cols, 4)
    d_y = torch.full((n_tok, rows), float("nan"), dtype=torch.float32, device="cuda")
    print("[gpu case] noalloc oversized scratch refused", flush=True)
    rc = L.swamp_qgemv_batched_noalloc(dtype, d_w.data_ptr(), raw.size, d_x.data_ptr(),
                                       d_y.data_ptr(), n_tok, rows, cols, 0, s)
    assert rc == EWORKSPACE
    torch.cuda.synchronize()
    assert torch.isnan(d_y).all().item()  # nothing written
