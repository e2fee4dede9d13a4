"""The C ABI: both libraries load, export every function include/*.h
declares, and reject bad arguments before touching a device.  CPU only (no
compute call is made)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header, prefix="swamp_"):
    text = open(os.path.join(REPO, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"[a-z0-9_]+)\s*\(", text)))


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_gpu_lib_exports_header(pkg):
    names = declared("swamp_qmm.h")
    assert set(names) == set(pkg.GPU_SYMBOLS)
    syms = exported(pkg.GPU_LIB_PATH)
    missing = [n for n in names if n not in syms]
    assert not missing, missing
    pkg.gpu_lib()  # dlopen + every signature binds


def test_gpu_lib_exports_gguf_header(pkg):
    names = declared("swamp_gguf.h")
    assert set(names) == set(pkg.GGUF_SYMBOLS)
    syms = exported(pkg.GPU_LIB_PATH)
    assert not [n for n in names if n not in syms]


def test_gpu_lib_exports_device_header(pkg):
    """The device-management functions the reference's bridge looks up by
    name in libswamp_gpu.so (swamp-gpu/src/lib.rs)."""
    names = declared("swamp_gpu.h", prefix="gpu_")
    assert set(names) == set(pkg.DEVICE_SYMBOLS)
    syms = exported(pkg.GPU_LIB_PATH)
    assert not [n for n in names if n not in syms]
    pkg.gpu_lib()


def test_gpu_lib_exports_nothing_else(pkg):
    """Only what the public headers declare is exported: the internal
    launchers and helpers are hidden (the HIP runtime's per-unit ids
    aside)."""
    public = (set(declared("swamp_qmm.h")) | set(declared("swamp_gguf.h")) |
              set(declared("swamp_gpu.h", prefix="gpu_")))
    extra = [n for n in exported(pkg.GPU_LIB_PATH)
             if n not in public and not n.startswith("__hip_cuid_")]
    assert not extra, extra


def test_stamps_library_is_the_product_plus_one_export(pkg):
    """libswamp_gpu_stamps.so (bench.py --gemv-stages) exports what the
    product does plus swamp_gemv_stage_stamps; the product does not export
    it (its stamps are compiled away)."""
    path = os.path.join(os.path.dirname(pkg.GPU_LIB_PATH), "libswamp_gpu_stamps.so")
    if not os.path.exists(path):
        pytest.skip("libswamp_gpu_stamps.so not built")
    prod = {n for n in exported(pkg.GPU_LIB_PATH) if not n.startswith("__hip_cuid_")}
    stamps = {n for n in exported(path) if not n.startswith("__hip_cuid_")}
    assert stamps - prod == {"swamp_gemv_stage_stamps"}
    assert prod <= stamps


def test_quant_lib_exports_header(pkg):
    names = declared("swamp_quant.h")
    assert set(names) == set(pkg.QUANT_SYMBOLS)
    syms = exported(pkg.QUANT_LIB_PATH)
    assert not [n for n in names if n not in syms]


def test_gpu_lib_has_gfx950_code(pkg):
    # the embedded offload bundle names its targets; only gfx950 is built
    data = open(pkg.GPU_LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", data))
    assert targets == {b"gfx950"}


def test_dtype_table_matches_oracle(pkg, orc):
    L, O = pkg.gpu_lib(), orc.lib()
    for code in list(range(0, 31)) + [99]:
        assert L.swamp_block_size(code) == O.or_block_size(code), code
        assert L.swamp_type_size(code) == O.or_type_size(code), code
        for n in (0, 1, 31, 32, 33, 256, 257, 4096 * 4096):
            assert L.swamp_nbytes_for(code, n) == O.or_nbytes_for(code, n)


def test_strerror(pkg):
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10, -11, -77):
        assert isinstance(pkg.strerror(code), str) and pkg.strerror(code)


def test_argument_validation_precedes_device(pkg):
    L = pkg.gpu_lib()
    fake = 0x10000  # never dereferenced: every call below fails validation
    # unsupported dtype (Q5_K = 13)
    assert L.swamp_qgemv(13, fake, 1 << 20, fake, fake, 4, 256, None) == pkg.EDTYPE
    # n_cols not a multiple of the block
    assert L.swamp_qgemv(pkg.Q4_K, fake, 1 << 20, fake, fake, 4, 255, None) == pkg.ESHAPE
    assert L.swamp_qgemv(pkg.Q4_0, fake, 1 << 20, fake, fake, 4, 48, None) == pkg.ESHAPE
    # weight buffer too small (BufferTooSmall / length assert)
    assert L.swamp_qgemv(pkg.Q4_0, fake, 100, fake, fake, 4, 64, None) == pkg.ESHAPE
    # null / misaligned
    assert L.swamp_qgemv(pkg.Q4_0, None, 1 << 20, fake, fake, 4, 64, None) == pkg.EINVAL
    assert L.swamp_qgemv(pkg.Q4_K, fake + 4, 1 << 20, fake, fake, 4, 256, None) == pkg.EINVAL
    assert L.swamp_qgemv(pkg.Q4_0, fake, 1 << 20, fake + 4, fake, 4, 64, None) == pkg.EINVAL
    assert L.swamp_qgemv_batched(pkg.Q4_0, fake, 1 << 20, fake, fake, -1, 4, 64, 0, None) == pkg.EINVAL
    assert L.swamp_qgemm(pkg.Q4_0, fake, 1 << 20, fake, pkg.F16, fake, 4, 4, 64, None) == pkg.EDTYPE
    assert L.swamp_qdequant(13, fake, 1 << 20, fake, 64, None) == pkg.EDTYPE
    # Q6_K: whole 256-blocks, 4-byte aligned rows base, enough bytes; no
    # accumulating batched form and no int8 GEMM
    assert L.swamp_qgemv(pkg.Q6_K, fake, 1 << 20, fake, fake, 4, 300, None) == pkg.ESHAPE
    assert L.swamp_qgemv(pkg.Q6_K, fake, 4 * 420 - 1, fake, fake, 4, 512, None) == pkg.ESHAPE
    assert L.swamp_qgemv(pkg.Q6_K, fake + 2, 1 << 20, fake, fake, 4, 512, None) == pkg.EINVAL
    assert L.swamp_qgemv_batched(pkg.Q6_K, fake, 1 << 20, fake, fake, 2, 4, 512, 1, None) == pkg.EDTYPE
    assert L.swamp_qgemm(pkg.Q6_K, fake, 1 << 20, fake, pkg.Q8_0, fake, 4, 4, 512, None) == pkg.EDTYPE
    assert L.swamp_qdequant(pkg.Q6_K, fake, 419, fake, 512, None) == pkg.ESHAPE
    # fused prologues: one item per lane (n_cols <= 32768, whole items)
    import ctypes
    one = lambda T, v: (T * 1)(v)
    def rms(dt, cols, norm=fake, x=fake, eps=1e-5):
        return L.swamp_qgemv_rmsnorm(1, one(ctypes.c_uint32, dt), one(ctypes.c_void_p, fake),
                                     one(ctypes.c_size_t, 1 << 30), one(ctypes.c_int, 4), x,
                                     norm, eps, one(ctypes.c_void_p, fake), cols, None)
    assert rms(pkg.Q4_0, 32832) == pkg.ESHAPE
    assert rms(pkg.Q4_0, 96) == pkg.ESHAPE and rms(pkg.Q4_0, 0) == pkg.ESHAPE
    assert rms(pkg.Q6_K, 256) == pkg.ESHAPE and rms(pkg.Q4_K, 320) == pkg.ESHAPE
    assert rms(pkg.Q4_0, 4096, norm=None) == pkg.EINVAL
    assert rms(pkg.Q4_0, 4096, norm=fake + 4) == pkg.EINVAL
    assert rms(13, 4096) == pkg.EDTYPE
    sw = lambda dt, cols, up=fake: L.swamp_qgemv_swiglu(dt, fake, 1 << 30, fake, up, fake, 4,
                                                        cols, 1, None)
    assert sw(pkg.Q8_0, 96) == pkg.ESHAPE and sw(pkg.Q8_0, 32832) == pkg.ESHAPE
    assert sw(pkg.Q6_K, 768) == pkg.ESHAPE and sw(pkg.Q4_K, 0) == pkg.ESHAPE
    assert sw(pkg.Q8_0, 4096, up=None) == pkg.EINVAL and sw(pkg.Q8_0, 4096, up=fake + 8) == pkg.EINVAL
    assert L.swamp_qdequant(pkg.Q4_0, fake, 35, fake, 64, None) == pkg.ESHAPE
    # bf16 dequant: weight dtypes only, whole blocks, aligned buffers
    dq16 = lambda dt, raw, rl, dst, n: L.swamp_qdequant_bf16(dt, raw, rl, dst, n, None)
    assert dq16(pkg.F32, fake, 1 << 20, fake, 64) == pkg.EDTYPE
    assert dq16(13, fake, 1 << 20, fake, 64) == pkg.EDTYPE
    assert dq16(pkg.Q4_0, fake, 35, fake, 64) == pkg.ESHAPE
    assert dq16(pkg.Q4_0, fake, 1 << 20, fake, 48) == pkg.ESHAPE
    assert dq16(pkg.Q4_K, fake, 1 << 20, fake, 288) == pkg.ESHAPE
    assert dq16(pkg.Q6_K, fake, 419, fake, 512) == pkg.ESHAPE
    assert dq16(pkg.Q4_0, fake + 2, 1 << 20, fake, 64) == pkg.EINVAL
    assert dq16(pkg.Q4_K, fake + 4, 1 << 20, fake, 256) == pkg.EINVAL
    assert dq16(pkg.Q6_K, fake + 1, 1 << 20, fake, 256) == pkg.EINVAL
    assert dq16(pkg.Q8_0, fake, 1 << 20, fake + 8, 64) == pkg.EINVAL
    assert dq16(pkg.Q8_0, None, 1 << 20, fake, 64) == pkg.EINVAL
    assert L.swamp_quantize_q8_0(fake, pkg.F32, fake, 33, None) == pkg.ESHAPE
    # activation producers: argument errors return before any device work
    rr = lambda ot, t, c, x=fake, w=fake, o=fake: L.swamp_rmsnorm_rows(x, w, 1e-5, o, ot, t, c,
                                                                       None)
    assert rr(pkg.F32, 4, 4098) == pkg.ESHAPE and rr(pkg.Q8_0, 4, 4096) == pkg.EDTYPE
    assert rr(pkg.F32, -1, 4096) == pkg.EINVAL and rr(pkg.F32, 4, -4) == pkg.EINVAL
    assert rr(pkg.F32, 4, 4096, x=None) == pkg.EINVAL and rr(pkg.F32, 4, 4096, w=fake + 4) == pkg.EINVAL
    assert rr(pkg.F32, 4, 4096, o=fake + 8) == pkg.EINVAL and rr(pkg.BF16, 4, 4096, o=fake + 4) == pkg.EINVAL
    assert rr(pkg.F32, 0, 4096) == pkg.OK and rr(pkg.BF16, 4, 0, x=None) == pkg.OK
    sg = lambda ot, n, g=fake, u=fake, o=fake: L.swamp_swiglu(g, u, o, ot, n, None)
    assert sg(pkg.F32, 14338) == pkg.ESHAPE and sg(pkg.F16, 14336) == pkg.EDTYPE
    assert sg(pkg.BF16, 14336, u=None) == pkg.EINVAL and sg(pkg.F32, 14336, g=fake + 4) == pkg.EINVAL
    assert sg(pkg.BF16, 14336, o=fake + 2) == pkg.EINVAL and sg(pkg.F32, 0, g=None) == pkg.OK
    n = 9
    dts = (ctypes.c_uint32 * n)(*([pkg.Q4_0] * n))
    assert L.swamp_qgemv_multi(n, dts, None, None, None, fake, None, 64, None) == pkg.EINVAL


def test_legacy_exports_null_behaviour(pkg):
    L = pkg.gpu_lib()
    # swamp_gemv_q8_vnni: null or k <= 0 -> 0.0 (lib.rs:458)
    assert L.swamp_gemv_q8_vnni(None, None, 64, 1.0) == 0.0
    buf = np.zeros(8, np.int8)
    assert L.swamp_gemv_q8_vnni(buf.ctypes.data, buf.ctypes.data, 0, 1.0) == 0.0
    # swamp_fused_gemv_q4k: null -> silent return; n_cols % 256 -> silent return
    out = np.full(4, 7.0, np.float32)
    L.swamp_fused_gemv_q4k(None, None, out.ctypes.data, 4, 256)
    L.swamp_fused_gemv_q4k(buf.ctypes.data, buf.ctypes.data, out.ctypes.data, 4, 100)
    assert out.tolist() == [7.0] * 4
