"""ctypes binding of libswamp_gpu.so / libswamp_quant.so.

Mirrors the loader of the reference's GPU bridge (swamp-gpu/src/lib.rs:30-54:
one-time library load, symbol lookup, integer return codes mapped to an error
type) for the quantized-matmul C ABI in include/swamp_qmm.h and the host
quantizers in include/swamp_quant.h.  Device buffers are passed as integer
addresses (for example torch.Tensor.data_ptr()); nothing here computes on the
CPU except the host quantizers, which only prepare weight bytes.

The directory name contains a dot, so import it by path:
    spec = importlib.util.spec_from_file_location("llamanyon_rs_amd", ".../__init__.py")
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Sequence

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
GPU_LIB_PATH = os.path.join(PKG_DIR, "libswamp_gpu.so")
QUANT_LIB_PATH = os.path.join(PKG_DIR, "libswamp_quant.so")

# GGML dtype codes (swamp-gguf/src/dtype.rs:10-40)
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 14, 30
DTYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K",
               BF16: "BF16"}
BLOCK = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}
TYPE_SIZE = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210}

# return codes (include/swamp_qmm.h, include/swamp_gguf.h)
OK, EINVAL, EDTYPE, ESHAPE, ELAUNCH, ENODEVICE, EWORKSPACE = 0, -1, -2, -3, -4, -5, -6
EIO, EMAGIC, EVERSION, ENOTFOUND, ETENSOR = -7, -8, -9, -10, -11
MULTI_MAX = 8

# Every symbol include/swamp_qmm.h declares.
GPU_SYMBOLS = (
    "swamp_gpu_init", "swamp_strerror", "swamp_block_size", "swamp_type_size",
    "swamp_nbytes_for", "swamp_qdequant", "swamp_qdequant_bf16", "swamp_qgemv", "swamp_qgemv_f16x", "swamp_qgemv_multi",
    "swamp_qgemv_rmsnorm", "swamp_qgemv_swiglu",
    "swamp_qgemv_batched", "swamp_qgemm", "swamp_rmsnorm_rows", "swamp_swiglu",
    "swamp_quantize_q8_0", "swamp_fused_gemv_q4k", "swamp_gemv_q8_vnni",
    "swamp_qgemv_batched_workspace", "swamp_qgemm_workspace", "swamp_workspace_reserve",
    "swamp_qgemv_batched_noalloc", "swamp_qgemv_many",
)
# Every symbol include/swamp_gguf.h declares (also in libswamp_gpu.so).
GGUF_SYMBOLS = (
    "swamp_gguf_open", "swamp_gguf_close", "swamp_gguf_version", "swamp_gguf_n_tensors",
    "swamp_gguf_n_kv", "swamp_gguf_data_offset", "swamp_gguf_file_size",
    "swamp_gguf_tensor_info", "swamp_gguf_find", "swamp_gguf_tensor_raw", "swamp_gguf_upload",
    "swamp_gguf_meta_type", "swamp_gguf_meta_u32", "swamp_gguf_meta_u64", "swamp_gguf_meta_f32",
    "swamp_gguf_meta_str",
)
# Every symbol include/swamp_gpu.h declares: the device-management functions
# the reference's bridge resolves by name (swamp-gpu/src/lib.rs:62-71,
# :110-142, :239-347, :599-665).
DEVICE_SYMBOLS = (
    "gpu_init", "gpu_alloc", "gpu_free", "gpu_copy_to_device", "gpu_copy_to_host", "gpu_sync",
    "gpu_stream_create", "gpu_stream_destroy", "gpu_stream_synchronize",
    "gpu_copy_to_device_async", "gpu_copy_to_host_async", "gpu_event_create",
    "gpu_event_record", "gpu_event_synchronize", "gpu_event_elapsed_ms", "gpu_event_destroy",
)
QUANT_SYMBOLS = (
    "swamp_f32_to_f16", "swamp_f32_to_bf16", "swamp_f32_to_bf16_array",
    "swamp_fill_normal", "swamp_quantize", "swamp_synth_quantized",
)


class GpuError(RuntimeError):
    """GpuError::{LibLoad, Symbol, KernelError} of swamp-gpu/src/lib.rs:16-28."""

    def __init__(self, code: int, what: str = ""):
        self.code = code
        super().__init__(f"{what}: error {code} ({strerror(code) if _gpu else 'library not loaded'})")


_gpu: Optional[ctypes.CDLL] = None
_quant: Optional[ctypes.CDLL] = None

c_size = ctypes.c_size_t
c_vp = ctypes.c_void_p


def build(force: bool = False) -> None:
    """Compile both libraries in-tree with the package Makefile."""
    cmd = ["make", "-C", PKG_DIR, "-j8"]
    if force:
        subprocess.run(["make", "-C", PKG_DIR, "clean"], check=True, stdout=subprocess.DEVNULL)
    subprocess.run(cmd, check=True)


def gpu_lib() -> ctypes.CDLL:
    """Load libswamp_gpu.so once (OnceLock semantics of swamp-gpu/src/lib.rs:30)."""
    global _gpu
    if _gpu is not None:
        return _gpu
    if not os.path.exists(GPU_LIB_PATH):
        raise GpuError(ENODEVICE, f"{GPU_LIB_PATH} not built (run build())")
    lib = ctypes.CDLL(GPU_LIB_PATH)
    u32, i32 = ctypes.c_uint32, ctypes.c_int
    sig = {
        "swamp_gpu_init": (i32, []),
        "swamp_strerror": (ctypes.c_char_p, [i32]),
        "swamp_block_size": (c_size, [u32]),
        "swamp_type_size": (c_size, [u32]),
        "swamp_nbytes_for": (c_size, [u32, c_size]),
        "swamp_qdequant": (i32, [u32, c_vp, c_size, c_vp, c_size, c_vp]),
        "swamp_qdequant_bf16": (i32, [u32, c_vp, c_size, c_vp, c_size, c_vp]),
        "swamp_qgemv": (i32, [u32, c_vp, c_size, c_vp, c_vp, i32, i32, c_vp]),
        "swamp_qgemv_f16x": (i32, [u32, c_vp, c_size, c_vp, c_vp, i32, i32, c_vp]),
        "swamp_qgemv_many": (i32, [i32, ctypes.POINTER(u32), ctypes.POINTER(c_vp),
                                   ctypes.POINTER(c_size), ctypes.POINTER(i32),
                                   ctypes.POINTER(i32), ctypes.POINTER(c_vp),
                                   ctypes.POINTER(c_vp), c_vp]),
        "swamp_qgemv_multi": (i32, [i32, ctypes.POINTER(u32), ctypes.POINTER(c_vp),
                                    ctypes.POINTER(c_size), ctypes.POINTER(i32), c_vp,
                                    ctypes.POINTER(c_vp), i32, c_vp]),
        "swamp_qgemv_rmsnorm": (i32, [i32, ctypes.POINTER(u32), ctypes.POINTER(c_vp),
                                      ctypes.POINTER(c_size), ctypes.POINTER(i32), c_vp, c_vp,
                                      ctypes.c_float, ctypes.POINTER(c_vp), i32, c_vp]),
        "swamp_qgemv_swiglu": (i32, [u32, c_vp, c_size, c_vp, c_vp, c_vp, i32, i32, i32, c_vp]),
        "swamp_qgemv_batched": (i32, [u32, c_vp, c_size, c_vp, c_vp, i32, i32, i32, i32, c_vp]),
        "swamp_qgemm": (i32, [u32, c_vp, c_size, c_vp, u32, c_vp, i32, i32, i32, c_vp]),
        "swamp_rmsnorm_rows": (i32, [c_vp, c_vp, ctypes.c_float, c_vp, u32, i32, i32, c_vp]),
        "swamp_swiglu": (i32, [c_vp, c_vp, c_vp, u32, c_size, c_vp]),
        "swamp_quantize_q8_0": (i32, [c_vp, u32, c_vp, c_size, c_vp]),
        "swamp_fused_gemv_q4k": (None, [c_vp, c_vp, c_vp, i32, i32]),
        "swamp_qgemv_batched_workspace": (c_size, [u32, i32, i32, i32, i32]),
        "swamp_qgemm_workspace": (c_size, [u32, u32, i32, i32, i32]),
        "swamp_workspace_reserve": (i32, [c_vp, c_size]),
        "swamp_qgemv_batched_noalloc": (i32, [u32, c_vp, c_size, c_vp, c_vp, i32, i32, i32, i32,
                                              c_vp]),
        "swamp_gemv_q8_vnni": (ctypes.c_float, [c_vp, c_vp, i32, ctypes.c_float]),
        # GGUF reader (include/swamp_gguf.h)
        "swamp_gguf_open": (i32, [ctypes.c_char_p, ctypes.POINTER(c_vp)]),
        "swamp_gguf_close": (None, [c_vp]),
        "swamp_gguf_version": (u32, [c_vp]),
        "swamp_gguf_n_tensors": (ctypes.c_int64, [c_vp]),
        "swamp_gguf_n_kv": (ctypes.c_int64, [c_vp]),
        "swamp_gguf_data_offset": (ctypes.c_uint64, [c_vp]),
        "swamp_gguf_file_size": (ctypes.c_uint64, [c_vp]),
        "swamp_gguf_tensor_info": (i32, [c_vp, ctypes.c_int64, ctypes.POINTER(ctypes.c_char_p),
                                         ctypes.POINTER(u32), ctypes.POINTER(i32),
                                         ctypes.POINTER(ctypes.c_uint64),
                                         ctypes.POINTER(ctypes.c_uint64),
                                         ctypes.POINTER(ctypes.c_uint64)]),
        "swamp_gguf_find": (ctypes.c_int64, [c_vp, ctypes.c_char_p]),
        "swamp_gguf_tensor_raw": (i32, [c_vp, ctypes.c_int64, ctypes.POINTER(c_vp),
                                        ctypes.POINTER(c_size)]),
        "swamp_gguf_upload": (i32, [c_vp, ctypes.c_int64, c_vp, c_size, c_vp]),
        "swamp_gguf_meta_type": (i32, [c_vp, ctypes.c_char_p, ctypes.POINTER(u32)]),
        "swamp_gguf_meta_u32": (i32, [c_vp, ctypes.c_char_p, ctypes.POINTER(u32)]),
        "swamp_gguf_meta_u64": (i32, [c_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
        "swamp_gguf_meta_f32": (i32, [c_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)]),
        "swamp_gguf_meta_str": (i32, [c_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p),
                                      ctypes.POINTER(c_size)]),
        # device management (include/swamp_gpu.h)
        "gpu_init": (i32, []),
        "gpu_alloc": (c_vp, [c_size]),
        "gpu_free": (None, [c_vp]),
        "gpu_copy_to_device": (i32, [c_vp, c_vp, c_size]),
        "gpu_copy_to_host": (i32, [c_vp, c_vp, c_size]),
        "gpu_sync": (i32, []),
        "gpu_stream_create": (c_vp, []),
        "gpu_stream_destroy": (None, [c_vp]),
        "gpu_stream_synchronize": (i32, [c_vp]),
        "gpu_copy_to_device_async": (i32, [c_vp, c_vp, c_size, c_vp]),
        "gpu_copy_to_host_async": (i32, [c_vp, c_vp, c_size, c_vp]),
        "gpu_event_create": (c_vp, []),
        "gpu_event_record": (i32, [c_vp, c_vp]),
        "gpu_event_synchronize": (i32, [c_vp]),
        "gpu_event_elapsed_ms": (ctypes.c_float, [c_vp, c_vp]),
        "gpu_event_destroy": (None, [c_vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _gpu = lib
    return lib


def quant_lib() -> ctypes.CDLL:
    global _quant
    if _quant is not None:
        return _quant
    if not os.path.exists(QUANT_LIB_PATH):
        raise GpuError(ENODEVICE, f"{QUANT_LIB_PATH} not built (run build())")
    lib = ctypes.CDLL(QUANT_LIB_PATH)
    u32, i32, u64 = ctypes.c_uint32, ctypes.c_int, ctypes.c_uint64
    sig = {
        "swamp_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
        "swamp_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
        "swamp_f32_to_bf16_array": (None, [c_vp, c_vp, c_size]),
        "swamp_fill_normal": (i32, [u64, ctypes.c_float, c_vp, c_size, c_size, i32]),
        "swamp_quantize": (i32, [u32, c_vp, c_vp, c_size, c_size, i32]),
        "swamp_synth_quantized": (i32, [u32, u64, ctypes.c_float, c_vp, c_size, c_size, i32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _quant = lib
    return lib


def strerror(code: int) -> str:
    return gpu_lib().swamp_strerror(code).decode()


def _check(rc: int, what: str) -> None:
    if rc != OK:
        raise GpuError(rc, what)


def row_bytes(dtype: int, n_cols: int) -> int:
    return n_cols // BLOCK[dtype] * TYPE_SIZE[dtype]


def nbytes(dtype: int, n_rows: int, n_cols: int) -> int:
    return n_rows * row_bytes(dtype, n_cols)


# ---------------------------------------------------------------- device API

def init() -> None:
    _check(gpu_lib().swamp_gpu_init(), "swamp_gpu_init")


def qdequant(dtype: int, d_raw: int, raw_len: int, d_dst: int, n: int, stream: int = 0) -> None:
    _check(gpu_lib().swamp_qdequant(dtype, d_raw, raw_len, d_dst, n, stream), "swamp_qdequant")


def qdequant_bf16(dtype: int, d_raw: int, raw_len: int, d_dst: int, n: int,
                  stream: int = 0) -> None:
    """n bf16 values (uint16 bits) at d_dst: swamp_qdequant's values rounded
    to nearest even."""
    _check(gpu_lib().swamp_qdequant_bf16(dtype, d_raw, raw_len, d_dst, n, stream),
           "swamp_qdequant_bf16")


def qgemv(dtype: int, d_w: int, w_len: int, d_x: int, d_y: int, n_rows: int, n_cols: int,
          stream: int = 0) -> None:
    _check(gpu_lib().swamp_qgemv(dtype, d_w, w_len, d_x, d_y, n_rows, n_cols, stream), "swamp_qgemv")


def qgemv_f16x(dtype: int, d_w: int, w_len: int, d_x: int, d_y: int, n_rows: int, n_cols: int,
               stream: int = 0) -> None:
    """swamp_qgemv with x rounded to fp16 inside the kernel (faster, ~1e-5)."""
    _check(gpu_lib().swamp_qgemv_f16x(dtype, d_w, w_len, d_x, d_y, n_rows, n_cols, stream),
           "swamp_qgemv_f16x")


def qgemv_multi(dtypes: Sequence[int], d_ws: Sequence[int], w_lens: Sequence[int],
                row_counts: Sequence[int], d_x: int, d_ys: Sequence[int], n_cols: int,
                stream: int = 0) -> None:
    n = len(dtypes)
    u32s = (ctypes.c_uint32 * n)(*dtypes)
    ws = (c_vp * n)(*d_ws)
    lens = (c_size * n)(*w_lens)
    rows = (ctypes.c_int * n)(*row_counts)
    ys = (c_vp * n)(*d_ys)
    _check(gpu_lib().swamp_qgemv_multi(n, u32s, ws, lens, rows, d_x, ys, n_cols, stream),
           "swamp_qgemv_multi")


def qgemv_many(dtypes: Sequence[int], d_ws: Sequence[int], w_lens: Sequence[int],
               n_rows: Sequence[int], n_cols: Sequence[int], d_xs: Sequence[int],
               d_ys: Sequence[int], stream: int = 0) -> None:
    """forward_gemvs: several GEMVs, each with its own x and shape, one call."""
    n = len(dtypes)
    _check(gpu_lib().swamp_qgemv_many(n, (ctypes.c_uint32 * n)(*dtypes), (c_vp * n)(*d_ws),
                                      (c_size * n)(*w_lens), (ctypes.c_int * n)(*n_rows),
                                      (ctypes.c_int * n)(*n_cols), (c_vp * n)(*d_xs),
                                      (c_vp * n)(*d_ys), stream), "swamp_qgemv_many")


def qgemv_rmsnorm(dtypes: Sequence[int], d_ws: Sequence[int], w_lens: Sequence[int],
                  row_counts: Sequence[int], d_x: int, d_norm_w: int, eps: float,
                  d_ys: Sequence[int], n_cols: int, stream: int = 0) -> None:
    n = len(dtypes)
    u32s = (ctypes.c_uint32 * n)(*dtypes)
    ws = (c_vp * n)(*d_ws)
    lens = (c_size * n)(*w_lens)
    rows = (ctypes.c_int * n)(*row_counts)
    ys = (c_vp * n)(*d_ys)
    _check(gpu_lib().swamp_qgemv_rmsnorm(n, u32s, ws, lens, rows, d_x, d_norm_w, eps, ys, n_cols,
                                         stream), "swamp_qgemv_rmsnorm")


def qgemv_swiglu(dtype: int, d_w: int, w_len: int, d_gate: int, d_up: int, d_y: int,
                 n_rows: int, n_cols: int, accumulate: bool = False, stream: int = 0) -> None:
    _check(gpu_lib().swamp_qgemv_swiglu(dtype, d_w, w_len, d_gate, d_up, d_y, n_rows, n_cols,
                                        1 if accumulate else 0, stream), "swamp_qgemv_swiglu")


def qgemv_batched(dtype: int, d_w: int, w_len: int, d_x: int, d_y: int, n_tok: int,
                  n_rows: int, n_cols: int, accumulate: bool = False, stream: int = 0) -> None:
    _check(gpu_lib().swamp_qgemv_batched(dtype, d_w, w_len, d_x, d_y, n_tok, n_rows, n_cols,
                                         1 if accumulate else 0, stream), "swamp_qgemv_batched")


def qgemv_batched_noalloc(dtype: int, d_w: int, w_len: int, d_x: int, d_y: int, n_tok: int,
                          n_rows: int, n_cols: int, accumulate: bool = False,
                          stream: int = 0) -> None:
    """swamp_qgemv_batched without any allocation (fixed 32 MiB scratch per GPU)."""
    _check(gpu_lib().swamp_qgemv_batched_noalloc(dtype, d_w, w_len, d_x, d_y, n_tok, n_rows,
                                                 n_cols, 1 if accumulate else 0, stream),
           "swamp_qgemv_batched_noalloc")


def qgemm(dtype: int, d_w: int, w_len: int, d_x: int, x_type: int, d_y: int, m: int,
          n_rows: int, n_cols: int, stream: int = 0) -> None:
    _check(gpu_lib().swamp_qgemm(dtype, d_w, w_len, d_x, x_type, d_y, m, n_rows, n_cols, stream),
           "swamp_qgemm")


def rmsnorm_rows(d_x: int, d_norm_w: int, eps: float, d_out: int, out_type: int, n_tok: int,
                 n_cols: int, stream: int = 0) -> None:
    """RMSNorm of n_tok rows (ops.rs:188-201) into fp32 or bf16 (the GEMM's x)."""
    _check(gpu_lib().swamp_rmsnorm_rows(d_x, d_norm_w, eps, d_out, out_type, n_tok, n_cols,
                                        stream), "swamp_rmsnorm_rows")


def swiglu(d_gate: int, d_up: int, d_out: int, out_type: int, n: int, stream: int = 0) -> None:
    """silu(gate) * up (ops.rs:203-214) into fp32 or bf16."""
    _check(gpu_lib().swamp_swiglu(d_gate, d_up, d_out, out_type, n, stream), "swamp_swiglu")


def workspace_reserve(stream: int, n_bytes: int) -> None:
    """Make the stream's scratch buffer at least n_bytes long now."""
    _check(gpu_lib().swamp_workspace_reserve(stream, n_bytes), "swamp_workspace_reserve")


def quantize_q8_0(d_x: int, x_type: int, d_q: int, n: int, stream: int = 0) -> None:
    _check(gpu_lib().swamp_quantize_q8_0(d_x, x_type, d_q, n, stream), "swamp_quantize_q8_0")


# ---------------------------------------------------------- host preparation

def _np():
    import numpy as np
    return np


def synth_quantized(dtype: int, seed: int, sigma: float, n_rows: int, n_cols: int,
                    n_threads: int = 0):
    """N(0, sigma^2) weights quantized to dtype blocks (numpy uint8 array)."""
    np = _np()
    out = np.empty(nbytes(dtype, n_rows, n_cols), dtype=np.uint8)
    _check(quant_lib().swamp_synth_quantized(dtype, seed, sigma, out.ctypes.data, n_rows,
                                             n_cols, n_threads), "swamp_synth_quantized")
    return out


def fill_normal(seed: int, sigma: float, n_rows: int, n_cols: int, n_threads: int = 0):
    np = _np()
    out = np.empty((n_rows, n_cols), dtype=np.float32)
    _check(quant_lib().swamp_fill_normal(seed, sigma, out.ctypes.data, n_rows, n_cols, n_threads),
           "swamp_fill_normal")
    return out


def quantize(dtype: int, src, n_threads: int = 0):
    np = _np()
    src = np.ascontiguousarray(src, dtype=np.float32)
    rows, cols = src.shape
    out = np.empty(nbytes(dtype, rows, cols), dtype=np.uint8)
    _check(quant_lib().swamp_quantize(dtype, src.ctypes.data, out.ctypes.data, rows, cols,
                                      n_threads), "swamp_quantize")
    return out


def to_bf16_bits(src):
    """float32 array -> uint16 bf16 bits (round to nearest even)."""
    np = _np()
    src = np.ascontiguousarray(src, dtype=np.float32)
    out = np.empty(src.shape, dtype=np.uint16)
    quant_lib().swamp_f32_to_bf16_array(src.ctypes.data, out.ctypes.data, src.size)
    return out


class TensorInfo:
    """TensorInfo (swamp-gguf/src/tensor_info.rs:8-15): name, shape, dtype and
    the ABSOLUTE file offset (GgufFile::parse adds the data offset,
    mmap.rs:81-86), plus nbytes (tensor_info.rs:24-27)."""

    __slots__ = ("index", "name", "shape", "dtype", "offset", "nbytes")

    def __init__(self, index, name, shape, dtype, offset, nbytes):
        self.index, self.name, self.shape = index, name, shape
        self.dtype, self.offset, self.nbytes = dtype, offset, nbytes

    def n_elems(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    def __repr__(self) -> str:
        return f"TensorInfo({self.name!r}, shape={self.shape}, dtype={self.dtype}, offset={self.offset})"


class GgufFile:
    """GgufFile (swamp-gguf/src/mmap.rs:16-151) over the C reader of
    include/swamp_gguf.h: the file is mapped read-only; tensor bytes are
    handed out zero-copy (tensor_raw_bytes) or copied straight to a device
    buffer (upload).  Errors raise GpuError with the reader's code."""

    def __init__(self, path: str):
        lib = gpu_lib()
        h = c_vp()
        _check(lib.swamp_gguf_open(os.fsencode(path), ctypes.byref(h)), f"swamp_gguf_open({path})")
        self._h = h
        self._lib = lib
        self.version = lib.swamp_gguf_version(h)
        self.data_offset = lib.swamp_gguf_data_offset(h)
        self.file_size = lib.swamp_gguf_file_size(h)
        self.n_kv = lib.swamp_gguf_n_kv(h)
        self.tensors = [self._info(i) for i in range(lib.swamp_gguf_n_tensors(h))]

    def _info(self, i: int) -> TensorInfo:
        name = ctypes.c_char_p()
        dt = ctypes.c_uint32()
        nd = ctypes.c_int()
        dims = (ctypes.c_uint64 * 4)()
        off = ctypes.c_uint64()
        nb = ctypes.c_uint64()
        _check(self._lib.swamp_gguf_tensor_info(self._h, i, ctypes.byref(name), ctypes.byref(dt),
                                                ctypes.byref(nd), dims, ctypes.byref(off),
                                                ctypes.byref(nb)), "swamp_gguf_tensor_info")
        shape = [int(dims[d]) for d in range(min(4, nd.value))]
        return TensorInfo(i, name.value.decode("utf-8", "replace"), shape, dt.value, off.value,
                          nb.value)

    def close(self) -> None:
        if self._h:
            self._lib.swamp_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def n_tensors(self) -> int:
        return len(self.tensors)

    def tensor(self, name: str) -> Optional[TensorInfo]:
        i = self._lib.swamp_gguf_find(self._h, name.encode())
        return self.tensors[i] if i >= 0 else None

    def tensor_or_err(self, name: str) -> TensorInfo:
        i = self._lib.swamp_gguf_find(self._h, name.encode())
        _check(int(i) if i < 0 else OK, f"tensor {name!r}")
        return self.tensors[i]

    def tensor_raw_bytes(self, info: TensorInfo):
        """numpy uint8 view of the mapping (valid while the file is open)."""
        np = _np()
        p, n = c_vp(), c_size()
        _check(self._lib.swamp_gguf_tensor_raw(self._h, info.index, ctypes.byref(p),
                                               ctypes.byref(n)), f"tensor_raw_bytes({info.name})")
        if n.value == 0:
            return np.zeros(0, np.uint8)
        buf = (ctypes.c_uint8 * n.value).from_address(p.value)
        return np.frombuffer(buf, dtype=np.uint8)

    def upload(self, info: TensorInfo, d_dst: int, dst_len: int, stream: int = 0) -> None:
        _check(self._lib.swamp_gguf_upload(self._h, info.index, d_dst, dst_len, stream),
               f"upload({info.name})")

    def meta_type(self, key: str) -> Optional[int]:
        t = ctypes.c_uint32()
        rc = self._lib.swamp_gguf_meta_type(self._h, key.encode(), ctypes.byref(t))
        return t.value if rc == OK else None

    def get_u32(self, key: str) -> int:
        v = ctypes.c_uint32()
        _check(self._lib.swamp_gguf_meta_u32(self._h, key.encode(), ctypes.byref(v)), key)
        return v.value

    def get_u64(self, key: str) -> int:
        v = ctypes.c_uint64()
        _check(self._lib.swamp_gguf_meta_u64(self._h, key.encode(), ctypes.byref(v)), key)
        return v.value

    def get_f32(self, key: str) -> float:
        v = ctypes.c_float()
        _check(self._lib.swamp_gguf_meta_f32(self._h, key.encode(), ctypes.byref(v)), key)
        return v.value

    def get_str(self, key: str) -> str:
        p, n = ctypes.c_char_p(), c_size()
        _check(self._lib.swamp_gguf_meta_str(self._h, key.encode(), ctypes.byref(p),
                                             ctypes.byref(n)), key)
        return ctypes.string_at(p, n.value).decode("utf-8", "replace")

    def architecture(self) -> str:
        """Metadata::architecture (metadata.rs:286-290): general.architecture
        as a string, else "unknown"."""
        try:
            return self.get_str("general.architecture")
        except GpuError:
            return "unknown"
