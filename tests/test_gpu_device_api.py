"""The reference's bridge end to end through the C ABI alone, no torch:
buffers from gpu_alloc, a stream from gpu_stream_create, copies queued on
it, the GEMV on it, events around it (the call pattern of
swamp-engine/src/scheduler.rs:24-60, :104-190 with the attention kernels
replaced by swamp_qgemv), checked against the oracle."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_0, Q4_K = 2, 12


@pytest.fixture(scope="module")
def L(pkg):
    lib = pkg.gpu_lib()
    try:
        import torch
        if not torch.cuda.is_available():
            pytest.skip("no GPU")
    except ImportError:
        pass
    assert lib.gpu_init() == 0
    return lib


def test_device_api_round_trip_gemv(pkg, orc, L):
    print("[gpu case] device api: alloc / async copies / qgemv on a created stream", flush=True)
    rows, cols = 3000, 4096
    raw = pkg.synth_quantized(Q4_K, 0x5EED ^ 0xD1, 0.02, rows, cols)
    x = pkg.fill_normal(0xA11CE ^ 0xD1, 1.0, 1, cols)[0]
    y = np.full(rows, np.nan, np.float32)
    s = L.gpu_stream_create()
    assert s
    d_w, d_x, d_y = L.gpu_alloc(raw.size), L.gpu_alloc(x.nbytes), L.gpu_alloc(y.nbytes)
    assert d_w and d_x and d_y
    e0, e1 = L.gpu_event_create(), L.gpu_event_create()
    assert e0 and e1
    try:
        assert L.gpu_copy_to_device_async(d_w, raw.ctypes.data, raw.size, s) == 0
        assert L.gpu_copy_to_device_async(d_x, x.ctypes.data, x.nbytes, s) == 0
        assert L.gpu_event_record(e0, s) == 0
        assert L.swamp_qgemv(Q4_K, d_w, raw.size, d_x, d_y, rows, cols, s) == 0
        assert L.gpu_event_record(e1, s) == 0
        assert L.gpu_copy_to_host_async(y.ctypes.data, d_y, y.nbytes, s) == 0
        assert L.gpu_stream_synchronize(s) == 0
        assert L.gpu_event_synchronize(e1) == 0
        ms = L.gpu_event_elapsed_ms(e0, e1)
        assert 0.0 <= ms < 1000.0
        ref = orc.forward_linear(Q4_K, raw, x, rows, cols, 8)
        deq = orc.dequantize(Q4_K, raw, rows * cols).reshape(rows, cols)
        err = orc.normalized_error(y, ref, deq, x)
        print(f"[gpu case] device api gemv normalized error {err:.3e}", flush=True)
        assert err <= 1e-3
        # synchronous copies and the device-wide sync
        back = np.zeros_like(x)
        assert L.gpu_copy_to_host(back.ctypes.data, d_x, x.nbytes) == 0
        assert np.array_equal(back, x)
        x2 = 2 * x
        assert L.gpu_copy_to_device(d_x, x2.ctypes.data, x.nbytes) == 0
        assert L.swamp_qgemv(Q4_K, d_w, raw.size, d_x, d_y, rows, cols, None) == 0
        assert L.gpu_sync() == 0
        y2 = np.empty_like(y)
        assert L.gpu_copy_to_host(y2.ctypes.data, d_y, y.nbytes) == 0
        assert np.array_equal(y2, 2 * y)
    finally:
        L.gpu_event_destroy(e0)
        L.gpu_event_destroy(e1)
        for p in (d_w, d_x, d_y):
            L.gpu_free(p)
        L.gpu_stream_destroy(s)


def test_device_api_null_handles(L):
    # destroy / free of NULL is a no-op, as in the reference
    L.gpu_free(None)
    L.gpu_stream_destroy(None)
    L.gpu_event_destroy(None)
    # the default stream synchronizes
    assert L.gpu_stream_synchronize(None) == 0
