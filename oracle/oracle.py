"""ctypes wrapper of liboracle.so -- TEST INFRASTRUCTURE ONLY.

The oracle is a plain-C restatement of the reference's scalar CPU matmul
path (see swamp_oracle.h for the file:line each function follows).  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it,
and only as the checker or as the timed CPU baseline.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "liboracle.so")

_lib = None
c_size = ctypes.c_size_t
c_vp = ctypes.c_void_p


def build() -> None:
    subprocess.run(["make", "-C", ORACLE_DIR], check=True, stdout=subprocess.DEVNULL)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    _lib = _bind(ctypes.CDLL(LIB_PATH))
    return _lib


# Flags of the CPU-baseline build: optimised for the host it runs on, with
# no contraction and no fast-math, so the arithmetic stays the reference's
# (Rust never contracts a*b+c) and only the speed differs from liboracle.so.
NATIVE_FLAGS = ["-O3", "-march=native", "-std=c11", "-fPIC", "-shared", "-pthread",
                "-ffp-contract=off", "-fno-fast-math"]


def use_native_build() -> str:
    """Switch this module to a build of swamp_oracle.c made now, on this host,
    with NATIVE_FLAGS (bench.py's cpu_baseline: -march=native must be compiled
    on the CPU that runs it).  Returns a description of the build in use;
    keeps liboracle.so when no C compiler is found or the build fails."""
    global _lib
    import shutil
    import tempfile
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        lib()
        return "oracle/liboracle.so (-O2; no C compiler for a native build)"
    out = os.path.join(tempfile.mkdtemp(prefix="swamp_oracle_native_"), "liboracle_native.so")
    cmd = [cc] + NATIVE_FLAGS + ["-o", out, os.path.join(ORACLE_DIR, "swamp_oracle.c"), "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        lib()
        return "oracle/liboracle.so (-O2; native build failed: " + r.stderr.strip()[-200:] + ")"
    _lib = _bind(ctypes.CDLL(out))
    return os.path.basename(cc) + " " + " ".join(f for f in NATIVE_FLAGS if f not in
                                                  ("-fPIC", "-shared", "-pthread"))


def _bind(L: ctypes.CDLL) -> ctypes.CDLL:
    u32, i32, f32 = ctypes.c_uint32, ctypes.c_int, ctypes.c_float
    sig = {
        "or_block_size": (c_size, [u32]),
        "or_type_size": (c_size, [u32]),
        "or_nbytes_for": (c_size, [u32, c_size]),
        "or_f16_to_f32": (f32, [ctypes.c_uint16]),
        "or_f16_to_f32_array": (None, [c_vp, c_vp, c_size]),
        "or_f16_to_f32_hw_array": (i32, [c_vp, c_vp, c_size]),
        "or_bf16_to_f32": (f32, [ctypes.c_uint16]),
        "or_dequantize": (i32, [u32, c_vp, c_size, c_vp, c_size]),
        "or_unpack_scales_q4k": (None, [c_vp, c_vp, c_vp]),
        "or_fused_gemv_q4k": (i32, [c_vp, c_size, c_vp, c_size, c_vp, c_size, c_size, c_size]),
        "or_fused_gemv_q6k": (i32, [c_vp, c_size, c_vp, c_size, c_vp, c_size, c_size, c_size]),
        "or_q6k_f16_raw": (f32, [ctypes.c_uint16]),
        "or_fused_gemv_q4k_batched": (i32, [c_vp, c_vp, c_vp, c_size, c_size, c_size]),
        "or_fused_gemv_q4k_multi": (i32, [c_vp, c_vp, c_vp, c_vp, c_size, c_size]),
        "or_forward_linear": (i32, [u32, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_size,
                                    c_size, i32]),
        "or_forward_linear_batch": (i32, [u32, c_vp, c_size, c_vp, c_vp, c_size, c_size, c_size,
                                          i32]),
        "or_rmsnorm": (None, [c_vp, c_vp, c_vp, c_size, f32]),
        "or_silu": (None, [c_vp, c_size]),
        "or_mul_in_place": (None, [c_vp, c_vp, c_size]),
        "or_add_in_place": (None, [c_vp, c_vp, c_size]),
        "or_gemv_q8_dot": (f32, [c_vp, c_vp, i32, f32]),
        "or_xorshift64_i8": (None, [ctypes.POINTER(ctypes.c_uint64), c_vp, c_size]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def f16_to_f32(codes: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint16)
    out = np.empty(codes.shape, dtype=np.float32)
    lib().or_f16_to_f32_array(_p(codes), _p(out), codes.size)
    return out


def f16_to_f32_hw(codes: np.ndarray):
    codes = np.ascontiguousarray(codes, dtype=np.uint16)
    out = np.empty(codes.shape, dtype=np.float32)
    if lib().or_f16_to_f32_hw_array(_p(codes), _p(out), codes.size) != 0:
        return None
    return out


def dequantize(dtype: int, raw: np.ndarray, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    rc = lib().or_dequantize(dtype, _p(raw), raw.size, _p(out), n)
    if rc != 0:
        raise ValueError(f"or_dequantize rc={rc}")
    return out


def unpack_scales_q4k(sc12: bytes):
    sc = np.frombuffer(bytes(sc12), dtype=np.uint8).copy()
    s = np.empty(8, dtype=np.uint8)
    m = np.empty(8, dtype=np.uint8)
    lib().or_unpack_scales_q4k(_p(sc), _p(s), _p(m))
    return s, m


def fused_gemv_q4k(w: np.ndarray, x: np.ndarray, n_rows: int, n_cols: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(n_rows, dtype=np.float32)
    rc = lib().or_fused_gemv_q4k(_p(w), w.size, _p(x), x.size, _p(out), out.size, n_rows, n_cols)
    if rc != 0:
        raise ValueError(f"or_fused_gemv_q4k rc={rc}")
    return out


def fused_gemv_q6k(w: np.ndarray, x: np.ndarray, n_rows: int, n_cols: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(n_rows, dtype=np.float32)
    rc = lib().or_fused_gemv_q6k(_p(w), w.size, _p(x), x.size, _p(out), out.size, n_rows, n_cols)
    if rc != 0:
        raise ValueError(f"or_fused_gemv_q6k rc={rc}")
    return out


def q6k_f16_raw(code: int) -> float:
    return float(lib().or_q6k_f16_raw(code))


def fused_gemv_q4k_batched(w: np.ndarray, xs: np.ndarray, outs: np.ndarray, n_rows: int,
                           n_cols: int) -> None:
    """outs[t] += W xs[t] (accumulating kernel contract)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    assert xs.flags.c_contiguous and outs.flags.c_contiguous
    bs = xs.shape[0]
    xp = (c_vp * bs)(*[xs.ctypes.data + t * xs.strides[0] for t in range(bs)])
    op = (c_vp * bs)(*[outs.ctypes.data + t * outs.strides[0] for t in range(bs)])
    rc = lib().or_fused_gemv_q4k_batched(_p(w), xp, op, n_rows, n_cols, bs)
    if rc != 0:
        raise ValueError(f"or_fused_gemv_q4k_batched rc={rc}")


def fused_gemv_q4k_multi(ws, x: np.ndarray, row_counts, n_cols: int):
    ws = [np.ascontiguousarray(w, dtype=np.uint8) for w in ws]
    x = np.ascontiguousarray(x, dtype=np.float32)
    outs = [np.empty(r, dtype=np.float32) for r in row_counts]
    n = len(ws)
    rp = (c_vp * n)(*[w.ctypes.data for w in ws])
    op = (c_vp * n)(*[o.ctypes.data for o in outs])
    rc_arr = (c_size * n)(*row_counts)
    rc = lib().or_fused_gemv_q4k_multi(rp, _p(x), op, rc_arr, n, n_cols)
    if rc != 0:
        raise ValueError(f"or_fused_gemv_q4k_multi rc={rc}")
    return outs


def forward_linear(dtype: int, raw: np.ndarray, x: np.ndarray, n_rows: int, n_cols: int,
                   n_threads: int = 1) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(n_rows, dtype=np.float32)
    rc = lib().or_forward_linear(dtype, _p(raw), raw.size, _p(x), x.size, _p(out), out.size,
                                 n_rows, n_cols, n_threads)
    if rc != 0:
        raise ValueError(f"or_forward_linear rc={rc}")
    return out


def forward_linear_batch(dtype: int, raw: np.ndarray, xs: np.ndarray, n_rows: int, n_cols: int,
                         n_threads: int = 1) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    bs = xs.shape[0]
    outs = np.empty((bs, n_rows), dtype=np.float32)
    rc = lib().or_forward_linear_batch(dtype, _p(raw), raw.size, _p(xs), _p(outs), bs, n_rows,
                                       n_cols, n_threads)
    if rc != 0:
        raise ValueError(f"or_forward_linear_batch rc={rc}")
    return outs


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    assert x.size == w.size
    out = np.empty_like(x)
    lib().or_rmsnorm(_p(out), _p(x), _p(w), x.size, eps)
    return out


def silu(x: np.ndarray) -> np.ndarray:
    out = np.array(x, dtype=np.float32, copy=True, order="C")
    lib().or_silu(_p(out), out.size)
    return out


def mul_in_place(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    out = np.array(a, dtype=np.float32, copy=True, order="C")
    b = np.ascontiguousarray(b, dtype=np.float32)
    lib().or_mul_in_place(_p(out), _p(b), out.size)
    return out


def add_in_place(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    out = np.array(a, dtype=np.float32, copy=True, order="C")
    b = np.ascontiguousarray(b, dtype=np.float32)
    lib().or_add_in_place(_p(out), _p(b), out.size)
    return out


def gemv_q8_dot(w: np.ndarray, a: np.ndarray, scale: float) -> float:
    w = np.ascontiguousarray(w, dtype=np.int8)
    a = np.ascontiguousarray(a, dtype=np.int8)
    return float(lib().or_gemv_q8_dot(_p(w), _p(a), w.size, scale))


def xorshift64_i8(state: int, n: int):
    s = ctypes.c_uint64(state)
    out = np.empty(n, dtype=np.int8)
    lib().or_xorshift64_i8(ctypes.byref(s), _p(out), n)
    return out, s.value


def normalized_error(y: np.ndarray, y_ref: np.ndarray, w_deq: np.ndarray, x: np.ndarray):
    """max_r |y[r] - y_ref[r]| / (||W_r|| * ||x||), norms in float64.

    w_deq is [rows, K] (the oracle-dequantized weights), x is [K] or [T, K]
    with y [T, rows]."""
    wn = np.linalg.norm(w_deq.astype(np.float64), axis=1)
    x64 = np.atleast_2d(x).astype(np.float64)
    xn = np.linalg.norm(x64, axis=1)
    diff = np.abs(np.atleast_2d(y).astype(np.float64) - np.atleast_2d(y_ref).astype(np.float64))
    denom = xn[:, None] * wn[None, :]
    denom = np.where(denom == 0, 1.0, denom)
    return float((diff / denom).max())
