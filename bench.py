"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline workload (one "step"): the Llama-3-8B decode layer sweep in Q4_0 at
batch 1 -- five GEMVs y = W x, fp32 x ~ N(0,1), W ~ N(0,0.02) quantized to
Q4_0 on the host:
    fused QKV 6144x4096, O-proj 4096x4096, fused gate+up 28672x4096,
    down 4096x14336, lm_head 128256x4096.
value = algorithmic bytes of one step / wall time of one step (GB/s), with
the weights already resident in HBM.  Algorithmic bytes per matrix =
rows*K*18/32 (Q4_0 blocks) + K*4 (x) + rows*4 (y).

Several full copies of the weight set (> 2x the 256 MB Infinity Cache in
total) are rotated step by step so every weight byte comes from HBM.  Before
the W warm-up steps, untimed steps run for --settle seconds (0.3 by default)
so the card has reached the clock it holds under sustained load.

Also reported (outside the timed steps):
  * roofline of the dominant kernel (the Q4_0 GEMV on lm_head, 70% of the
    step's bytes): its algorithmic bytes / its mean launch duration, timed
    with HIP events recorded on the launch stream around each of its
    launches in a second run of the K steps (events between kernels slow
    the step, so the first run, which gives `value`, has none);
  * per-matrix GB/s (each matrix timed alone, outside the timed region);
  * the Q4_0 prefill GEMM at 2048 and 512 tokens (mean of 20 back-to-back
    calls after 10 untimed ones), with bf16
    activations (fraction of the 2.5 PFLOP/s dense bf16 peak) and with
    Q8_0-quantized activations on the int8 MFMA (quantizer included;
    fraction of the 5.0 POP/s dense int8 peak);
  * small_batch: the Llama-3-8B layer in Q4_K with the lm_head in Q8_0 at
    1, 4, 8 and 16 tokens (swamp_qgemv, swamp_qgemv_batched), each matrix
    timed alone and summed (GB/s, fraction of HBM peak, GFLOP/s), with its
    CPU lines (the reference's fused_gemv_q4k_scalar and batched_scalar,
    restated in C) at the same thread counts as cpu_baseline;
  * decode_70b: the Llama-3-70B layer in Q4_K with the lm_head in Q8_0 at
    batch 1, the same way;
  * prefill_70b: the 70B gate+up, down and QKV as 4096-token bf16 prefill
    GEMMs (fraction of the bf16 peak);
  * cpu_baseline: the reference's CPU matmul path (forward_linear fallback:
    dequantize the whole tensor on one thread, then a row-partitioned f32
    dot), restated in C and compiled here with -O3 -march=native
    -ffp-contract=off, timed on this host's cores on full steps at 6
    threads (the reference's pool) and at every thread of the host's share,
    with the CPU model.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--no-prefill] [--no-small-batch] [--no-70b] [--cpu-threads 6,max]
                       [--sweep] [--pmc-probe] [--pmc-gemm] [--pmc-batched N] [--pmc-decode]
                       [--gemv-stages] [--gemv-fixed-cost] [--mfma-probe]
--sweep adds one JSON line per extra workload after the main line: the
Q4_K small batch at 2, 17, 24, 32 and 64 tokens (2 as one GEMV, 17-64 in
token groups of 16) at 8B shapes, the 8B shapes in Q6_K, the activation
producers, the rest of the 70B prefill and the int8 prefill with Q4_K
weights.  --pmc-probe runs only the dominant kernel
and a copy of known size, for the rocprofv3 --pmc traffic measurement;
--pmc-gemm the same for the 2048-token gate+up prefill GEMM; --pmc-batched N
runs 5 small-batch launches of N tokens per 8B sweep matrix, --pmc-decode 5
launches of each Q4_0 decode matrix, for counter passes.
--gemv-stages times the stages inside each 8B decode GEMV launch (stage
stamps of libswamp_gpu_stamps.so), --gemv-fixed-cost the decode GEMV against
row count, --mfma-probe the matrix-core issue microbenchmark; each prints
one JSON line and nothing else.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import re
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA

DECODE_SHAPES = [              # (name, rows, K), Llama-3-8B, Q4_0
    ("qkv", 6144, 4096),
    ("o_proj", 4096, 4096),
    ("gate_up", 28672, 4096),
    ("down", 4096, 14336),
    ("lm_head", 128256, 4096),
]
PREFILL_SHAPES = [("gate_up", 28672, 4096), ("down", 4096, 14336), ("qkv", 6144, 4096)]
PREFILL_MS = (2048, 512)        # prompt lengths of the prefill GEMM lines
SEED = 0x5EED


def _load(name, path):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def alg_bytes_gemv(dtype_bytes_per_32, rows, k, n_tok=1):
    return rows * k * dtype_bytes_per_32 // 32 + n_tok * k * 4 + n_tok * rows * 4


class TimingEvent:
    """A HIP timing event created with hipEventDisableSystemFence: recording
    it writes a timestamp on the stream without the system-scope release
    (an L2 writeback and invalidate) that a default event performs, which
    would otherwise add several microseconds to the timed step.  It uses the
    HIP runtime torch has loaded (same soname), so torch's stream handle is
    valid for it; read it only after a device synchronize."""

    DISABLE_SYSTEM_FENCE = 0x20000000  # hipEventDisableSystemFence

    _hip = None

    def __init__(self):
        import ctypes
        if TimingEvent._hip is None:
            TimingEvent._hip = ctypes.CDLL("libamdhip64.so.7")
        self._ct = ctypes
        self.ev = ctypes.c_void_p()
        rc = self._hip.hipEventCreateWithFlags(ctypes.byref(self.ev), self.DISABLE_SYSTEM_FENCE)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")

    def record(self, stream_handle):
        rc = self._hip.hipEventRecord(self.ev, self._ct.c_void_p(stream_handle))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_ms(self, end):
        ms = self._ct.c_float()
        rc = self._hip.hipEventElapsedTime(self._ct.byref(ms), self.ev, end.ev)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return float(ms.value)

    def __del__(self):
        if TimingEvent._hip is not None and self.ev:
            TimingEvent._hip.hipEventDestroy(self.ev)


def traffic_from_profiles():
    """HBM bytes per launch of the GEMV kernel, from the committed rocprofv3
    PMC summary (FETCH_SIZE + WRITE_SIZE, scaled by a copy-kernel
    calibration); None when no such summary exists."""
    path = os.path.join(REPO, "profiles", "gemv_q4_0_llama3_8b_decode_traffic.md")
    try:
        with open(path) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read(), re.M)
        return float(m.group(1)) if m else None
    except OSError:
        return None


def cpu_model():
    """The host CPU's model name (lscpu's "Model name", from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads_available():
    """Threads this process may use: the host's share (OMP_NUM_THREADS where
    the host sets it) capped by the logical CPUs."""
    n = os.cpu_count() or 1
    try:
        share = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        share = 0
    return min(n, share) if share > 0 else n


def _cpu_oracle():
    orc = _load("swamp_oracle_py", os.path.join(REPO, "oracle", "oracle.py"))
    build = orc.use_native_build()
    return orc, build


def cpu_baseline(pkg, thread_counts, min_seconds=8.0):
    """The reference's CPU path (oracle restatement of forward_linear's
    dequantize-then-dot fallback, swamp-engine/src/linear.rs:68-88) on
    full decode steps, at each thread count; GB/s over the step's
    algorithmic bytes.  The oracle is compiled on this host with -O3
    -march=native -ffp-contract=off."""
    orc, build = _cpu_oracle()
    mats = []
    for i, (_, rows, k) in enumerate(DECODE_SHAPES):
        raw = pkg.synth_quantized(pkg.Q4_0, SEED ^ i, 0.02, rows, k)
        x = pkg.fill_normal(SEED ^ 0xA11CE ^ i, 1.0, 1, k)[0]
        mats.append((raw, x, rows, k))
    total = sum(alg_bytes_gemv(18, r, k) for _, _, r, k in mats)
    runs = []
    for nt in thread_counts:
        times = []
        t_start = time.perf_counter()
        while len(times) < 2 or time.perf_counter() - t_start < min_seconds:
            t0 = time.perf_counter()
            for raw, x, rows, k in mats:
                orc.forward_linear(pkg.Q4_0, raw, x, rows, k, nt)
            times.append(time.perf_counter() - t0)
        t = float(sum(times) / len(times))
        runs.append({"threads": nt, "value": round(total / t / 1e9, 4),
                     "seconds_per_step": round(t, 3), "reps": len(times)})
    best = max(runs, key=lambda r: r["value"])
    return {
        "value": best["value"],
        "unit": "GB/s",
        "cores": best["threads"],
        "kind": "port",
        "sample": (f"full decode steps (5 Q4_0 GEMVs, {total} algorithmic bytes each), "
                   f"at least {min_seconds:.0f} s per thread count; C restatement of "
                   "forward_linear's fallback: allocate rows*K f32, dequantize on one thread, "
                   "row-partitioned sequential f32 dot"),
        "model": cpu_model(),
        "nproc": os.cpu_count(),
        "threads_available": cpu_threads_available(),
        "build": build,
        "runs": runs,
    }


def cpu_small_batch(pkg, thread_counts, min_seconds=2.0):
    """CPU lines of the small batch, with the oracle build of cpu_baseline:
    the Q4_K scalar GEMV (fused_gemv_q4k_scalar, fused_gemv_q4k.rs:466-508,
    rows partitioned as linear.rs:28-47) at 1 token and the Q4_K small batch
    (batched_scalar, :650-698, rows partitioned as linear.rs:209-236) at 4,
    8 and 16 tokens, over the four 8B layer matrices (the lm_head is left
    out to bound the time); GB/s over their algorithmic bytes."""
    orc, build = _cpu_oracle()
    layer = [(n, r, k) for n, r, k in SWEEP_8B if n != "lm_head"]
    mats = [(pkg.synth_quantized(pkg.Q4_K, SEED ^ 0x900 ^ i, 0.02, r, k), r, k)
            for i, (_, r, k) in enumerate(layer)]

    def timed(fn):
        times = []
        t_start = time.perf_counter()
        while len(times) < 2 or time.perf_counter() - t_start < min_seconds:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return float(sum(times) / len(times)), len(times)

    lines = []
    for n_tok in (1, 4, 8, 16):
        xs = [pkg.fill_normal(SEED ^ 0xA00 ^ i, 1.0, n_tok, k) for i, (_, _, k) in enumerate(layer)]
        nbytes = sum(int(r * k * 144 // 256) + n_tok * k * 4 + n_tok * r * 4 for _, r, k in mats)
        runs = []
        for nt in thread_counts:
            if n_tok == 1:
                fn = lambda: [orc.forward_linear(pkg.Q4_K, raw, x[0], r, k, nt)
                              for (raw, r, k), x in zip(mats, xs)]
            else:
                fn = lambda: [orc.forward_linear_batch(pkg.Q4_K, raw, x, r, k, nt)
                              for (raw, r, k), x in zip(mats, xs)]
            t, reps = timed(fn)
            runs.append({"threads": nt, "GB/s": round(nbytes / t / 1e9, 4),
                         "seconds_per_call": round(t, 4), "reps": reps})
        lines.append({"path": "fused_gemv_q4k_scalar" if n_tok == 1 else "batched_scalar",
                      "n_tok": n_tok, "alg_bytes": nbytes, "runs": runs})
    return {"workload": "llama3-8b Q4_K layer (qkv, o_proj, gate_up, down), kind port",
            "model": cpu_model(), "build": build, "lines": lines}


def cpu_sweep(pkg, thread_counts, min_seconds=4.0):
    """The Q4_0 prefill as forward_linear per token (opt-in, --sweep):
    linear.rs:68-88 applied to each token (the reference's own batched Q4_0
    arm decodes the bytes as Q4_K, linear.rs:358), on a sample of tokens."""
    orc, build = _cpu_oracle()

    def timed(fn):
        times = []
        t_start = time.perf_counter()
        while len(times) < 2 or time.perf_counter() - t_start < min_seconds:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return float(sum(times) / len(times)), len(times)

    # Q4_0 prefill semantics: forward_linear per token, on a token sample
    sample = 2
    per = []
    for i, (name, rows, k) in enumerate(PREFILL_SHAPES):
        raw = pkg.synth_quantized(pkg.Q4_0, SEED ^ 0x100 ^ i, 0.02, rows, k)
        xs = pkg.fill_normal(SEED ^ 0x200 ^ i, 1.0, sample, k)
        nt = max(thread_counts)
        t, reps = timed(lambda: orc.forward_linear_batch(pkg.Q4_0, raw, xs, rows, k, nt))
        per_tok = t / sample
        per.append({"name": name, "rows": rows, "k": k, "threads": nt,
                    "seconds_per_token": round(per_tok, 4),
                    "TFLOP/s": round(2 * rows * k / per_tok / 1e12, 6),
                    "seconds_at_m": {str(m): round(per_tok * m, 1) for m in PREFILL_MS}})
    print(json.dumps({"cpu_sweep": "llama3-8b Q4_0 prefill as forward_linear per token "
                                   f"(sample of {sample} tokens per matrix, scaled to M)",
                      "model": cpu_model(), "build": build, "matrices": per}), flush=True)


SWEEP_8B = [("qkv", 6144, 4096), ("o_proj", 4096, 4096), ("gate_up", 28672, 4096),
            ("down", 4096, 14336), ("lm_head", 128256, 4096)]
SWEEP_70B = [("qkv", 10240, 8192), ("o_proj", 8192, 8192), ("gate_up", 57344, 8192),
             ("down", 8192, 28672), ("lm_head", 128256, 8192)]


def _timed(torch, stream, fn, reps=20):
    """Mean time (us) of `reps` back-to-back calls fn(i), after 3 untimed
    ones and a GPU sleep (so the timed calls do not queue behind them)."""
    for i in range(3):
        fn(i)
    torch.cuda.synchronize()
    torch.cuda._sleep(20_000_000)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def _copies(nbytes):
    """Weight copies rotated per matrix: enough that the matrices cycled
    through exceed twice the 256 MB Infinity Cache (at least 2, at most 8)."""
    return max(2, min(8, int(2 * 256e6 // nbytes) + 1))


def _check(pkg, rc, what):
    if rc != 0:
        raise pkg.GpuError(rc, what)


def layer_lines(pkg, torch, stream, lib, shapes, sigma, n_toks, seed):
    """One line per token count: each matrix of the layer (Q4_K; lm_head
    Q8_0) timed alone over rotated weight copies -- swamp_qgemv at 1 token,
    swamp_qgemv_batched above (the reference's fused_gemv_q4k /
    fused_gemv_q4k_batched calls of benchmark_q4k_batched.rs:70-108, y
    overwritten, which equals its zero-fill plus accumulate) -- then summed:
    GB/s over the algorithmic bytes (W + N K 4 + N rows 4) and GFLOP/s over
    2 N rows K (benchmark_q4k_batched.rs:92-94)."""
    s = stream.cuda_stream
    bpw = {pkg.Q4_K: 144 / 256, pkg.Q8_0: 34 / 32}
    mats = []
    for i, (name, rows, k) in enumerate(shapes):
        dt = pkg.Q8_0 if name == "lm_head" else pkg.Q4_K
        d0 = torch.from_numpy(pkg.synth_quantized(dt, seed ^ 0x300 ^ i, sigma, rows, k)).cuda()
        n_cp = _copies(rows * k * bpw[dt])
        mats.append((name, dt, rows, k, [d0] + [d0.clone() for _ in range(n_cp - 1)]))
    out = []
    for n_tok in n_toks:
        per, tot_b, tot_us = [], 0, 0.0
        for i, (name, dt, rows, k, ws) in enumerate(mats):
            x = torch.from_numpy(pkg.fill_normal(seed ^ 0x400 ^ i, 1.0, n_tok, k)).cuda()
            y = torch.empty((n_tok, rows), dtype=torch.float32, device="cuda")
            n_cp = len(ws)
            if n_tok == 1:
                fn = lambda c: _check(pkg, lib.swamp_qgemv(dt, ws[c % n_cp].data_ptr(),
                                                           ws[0].numel(), x.data_ptr(),
                                                           y.data_ptr(), rows, k, s),
                                      "swamp_qgemv")
            else:
                fn = lambda c: _check(pkg, lib.swamp_qgemv_batched(
                    dt, ws[c % n_cp].data_ptr(), ws[0].numel(), x.data_ptr(), y.data_ptr(),
                    n_tok, rows, k, 0, s), "swamp_qgemv_batched")
            us = _timed(torch, stream, fn)
            b = int(rows * k * bpw[dt]) + n_tok * k * 4 + n_tok * rows * 4
            per.append({"name": name, "dtype": pkg.DTYPE_NAMES[dt], "rows": rows, "k": k,
                        "us": round(us, 2), "GB/s": round(b / us / 1e3, 1)})
            tot_b += b
            tot_us += us
            del x, y
        flop = sum(2 * n_tok * r * k for _, _, r, k, _ in mats)
        out.append({"n_tok": n_tok, "alg_bytes": tot_b, "us": round(tot_us, 1),
                    "GB/s": round(tot_b / tot_us / 1e3, 1),
                    "frac_hbm_peak": round(tot_b / tot_us / 1e3 / HBM_PEAK_GBS, 4),
                    "GFLOP/s": round(flop / tot_us / 1e3, 1), "matrices": per})
    del mats
    return out


def gemm_route(torch, dtype_q6k, m, rows, k, x_name):
    """Which of the library's kernels a swamp_qgemm call runs, by the rule
    of swamp_gemm_dq_route (csrc/gemm_dq.hip): bf16 x takes the
    dequantize-once route (blocks_to_bf16 + gemm_bb) for Q6_K, and from 1024
    tokens for shapes whose 256 x 256 tiles fill more than half but not all
    of the CUs; else the fused dequant GEMM (gemm_bf16_kernel).  Q8_0 x runs
    the int8 GEMM."""
    if x_name != "bf16":
        return "gemm_i8 (int8 MFMA)"
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tiles = ((m + 255) // 256) * ((rows + 255) // 256)
    if dtype_q6k or (m >= 1024 and k >= 1024 and 2 * tiles > cus and tiles < cus):
        return "dequantize-once: blocks_to_bf16 + gemm_bb (plain bf16 MFMA GEMM)"
    return "fused dequant bf16 MFMA GEMM (gemm_bf16_kernel)"


def prefill_70b_lines(pkg, torch, np, stream, lib, names, m=4096):
    """The 4096-token bf16 prefill GEMM at 70B shapes (Q4_K weights): mean of
    5 calls after 3 untimed ones per matrix; TFLOP/s over 2 M rows K."""
    s = stream.cuda_stream
    per = []
    for i, (name, rows, k) in enumerate(SWEEP_70B):
        if name not in names:
            continue
        dt = pkg.Q8_0 if name == "lm_head" else pkg.Q4_K
        w = torch.from_numpy(pkg.synth_quantized(dt, SEED ^ 0x500 ^ i, 0.015, rows, k)).cuda()
        xb = torch.from_numpy(pkg.to_bf16_bits(
            pkg.fill_normal(SEED ^ 0x600 ^ i, 1.0, m, k)).view(np.int16)).cuda()
        y = torch.empty((m, rows), dtype=torch.float32, device="cuda")
        fn = lambda c: _check(pkg, lib.swamp_qgemm(dt, w.data_ptr(), w.numel(), xb.data_ptr(),
                                                   pkg.BF16, y.data_ptr(), m, rows, k, s),
                              "swamp_qgemm")
        us = _timed(torch, stream, fn, reps=5)
        tf = 2 * m * rows * k / us / 1e6
        per.append({"name": name, "m": m, "dtype": pkg.DTYPE_NAMES[dt], "rows": rows, "k": k,
                    "x": "bf16", "route": gemm_route(torch, dt == pkg.Q6_K, m, rows, k, "bf16"),
                    "us": round(us, 1), "TFLOP/s": round(tf, 1),
                    "frac_peak": round(tf / BF16_PEAK_TFLOPS, 4), "peak": BF16_PEAK_TFLOPS})
        del w, xb, y
    return per


def run_sweep(pkg, torch, np, stream, lib):
    """Extra lines (opt-in, --sweep): the small-batch Q4_K sweep at 8B shapes
    (lm_head Q8_0) for 2, 17, 24, 32 and 64 tokens (17-64 in token groups of
    16), the 8B shapes in Q6_K at 1, 2, 4, 16 and 32 tokens, the activation
    producers, the 70B O-projection and lm_head as 4096-token bf16 prefill
    GEMMs, and the 8B layer (without lm_head) as a 2048-token int8 GEMM with
    Q4_K and Q4_0 weights.  Each matrix is timed alone: 20 launches over
    rotated weight copies behind a GPU sleep; GB/s over the algorithmic
    bytes, TFLOP/s over 2*M*rows*K."""
    s = stream.cuda_stream
    bpw = {pkg.Q4_0: 18 / 32, pkg.Q4_K: 144 / 256, pkg.Q8_0: 34 / 32, pkg.Q6_K: 210 / 256}

    def timed(fn, reps=20):
        for i in range(3):
            fn(i)
        torch.cuda.synchronize()
        torch.cuda._sleep(20_000_000)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(reps):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    def weights_dev(dt, rows, k, seed, sigma, copies):
        raw = pkg.synth_quantized(dt, seed, sigma, rows, k)
        d0 = torch.from_numpy(raw).cuda()
        return [d0] + [d0.clone() for _ in range(copies - 1)]

    def check(rc, what):
        if rc != 0:
            raise pkg.GpuError(rc, what)

    # token counts beyond the main line's: 2 (two-token GEMV), 17-64 (token groups)
    for line in layer_lines(pkg, torch, stream, lib, SWEEP_8B, 0.02, (2, 17, 24, 32, 64), SEED):
        print(json.dumps({"sweep": "llama3-8b small-batch Q4_K (lm_head Q8_0)", **line}),
              flush=True)
    # every 8B matrix in Q6_K (Q4_K_M files keep lm_head and part of attn_v /
    # ffn_down in Q6_K): batch-1 decode, and small batches of 2, 4, 16 and 32
    # tokens (one pass each)
    for n_tok in (1, 2, 4, 16, 32):
        per, tot_b, tot_us = [], 0, 0.0
        for i, (name, rows, k) in enumerate(SWEEP_8B):
            dt = pkg.Q6_K
            copies = max(2, min(8, int(2 * 256e6 // (rows * k * bpw[dt])) + 1))
            ws = weights_dev(dt, rows, k, SEED ^ 0x700 ^ i, 0.02, copies)
            x = torch.from_numpy(pkg.fill_normal(SEED ^ 0x800 ^ i, 1.0, n_tok, k)).cuda()
            y = torch.empty((n_tok, rows), dtype=torch.float32, device="cuda")
            if n_tok == 1:
                fn = lambda c: check(lib.swamp_qgemv(dt, ws[c % copies].data_ptr(), ws[0].numel(),
                                                     x.data_ptr(), y.data_ptr(), rows, k, s),
                                     "swamp_qgemv")
            else:
                fn = lambda c: check(lib.swamp_qgemv_batched(
                    dt, ws[c % copies].data_ptr(), ws[0].numel(), x.data_ptr(), y.data_ptr(),
                    n_tok, rows, k, 0, s), "swamp_qgemv_batched")
            us = timed(fn)
            b = int(rows * k * bpw[dt]) + n_tok * k * 4 + n_tok * rows * 4
            per.append({"name": name, "dtype": "Q6_K", "rows": rows, "k": k, "us": round(us, 2),
                        "GB/s": round(b / us / 1e3, 1)})
            tot_b += b
            tot_us += us
            del ws, x, y
        print(json.dumps({"sweep": "llama3-8b decode/small-batch Q6_K", "n_tok": n_tok,
                          "alg_bytes": tot_b, "us": round(tot_us, 1),
                          "GB/s": round(tot_b / tot_us / 1e3, 1),
                          "frac_hbm_peak": round(tot_b / tot_us / 1e3 / HBM_PEAK_GBS, 4),
                          "matrices": per}), flush=True)
    # activation producers of the 8B prefill at 2048 tokens: RMSNorm rows and
    # SiLU(gate) * up, written as the GEMM's bf16 input
    # (input copies rotate so that more than 512 MB cycles through the cache)
    m, per = 2048, []
    for name, k in (("rmsnorm_rows", 4096), ("swiglu", 14336)):
        a0 = torch.from_numpy(pkg.fill_normal(SEED ^ 0x700, 1.0, m, k)).cuda()
        b = torch.from_numpy(pkg.fill_normal(SEED ^ 0x701, 1.0, m, k)).cuda()
        n_cp = max(3, -(-(512 << 20) // (m * k * 4)))
        a = [a0] + [a0.clone() for _ in range(n_cp - 1)]
        o = torch.empty((m, k), dtype=torch.int16, device="cuda")
        if name == "rmsnorm_rows":
            wn = b[0].contiguous()
            fn = lambda c: check(lib.swamp_rmsnorm_rows(a[c % n_cp].data_ptr(), wn.data_ptr(),
                                                        1e-5, o.data_ptr(), pkg.BF16, m, k, s),
                                 "swamp_rmsnorm_rows")
            nb = m * k * 4 + k * 4 + m * k * 2
        else:
            bl = [b] + [b.clone() for _ in range(n_cp - 1)]
            fn = lambda c: check(lib.swamp_swiglu(a[c % n_cp].data_ptr(),
                                                  bl[c % n_cp].data_ptr(), o.data_ptr(),
                                                  pkg.BF16, m * k, s), "swamp_swiglu")
            nb = 2 * m * k * 4 + m * k * 2
        us = timed(fn)
        per.append({"name": name, "m": m, "k": k, "us": round(us, 2), "bytes": nb,
                    "GB/s": round(nb / us / 1e3, 1),
                    "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)})
        a = b = bl = wn = None
        del a0, o
    print(json.dumps({"sweep": "llama3-8b prefill activation producers -> bf16, 2048 tokens",
                      "kernels": per}), flush=True)
    # 70B prefill, 4096 tokens, bf16 activations, Q4_K weights (lm_head Q8_0):
    # the matrices the main line leaves out
    print(json.dumps({"sweep": "llama3-70b prefill Q4_K (lm_head Q8_0) x bf16, 4096 tokens",
                      "matrices": prefill_70b_lines(pkg, torch, np, stream, lib,
                                                    ("o_proj", "lm_head"))}), flush=True)
    # 8B prefill, 2048 tokens, Q4_K weights on the int8 MFMA against Q8_0 x
    # (quantizer included), beside the same calls with Q4_0 weights
    m = 2048
    per = []
    for i, (name, rows, k) in enumerate(SWEEP_8B[:4]):
        x = torch.from_numpy(pkg.fill_normal(SEED ^ 0x700 ^ i, 1.0, m, k)).cuda()
        xq = torch.empty(m * k // 32 * 34, dtype=torch.uint8, device="cuda")
        y = torch.empty((m, rows), dtype=torch.float32, device="cuda")
        for dt in (pkg.Q4_K, pkg.Q4_0):
            ws = weights_dev(dt, rows, k, SEED ^ 0x800 ^ i, 0.02, 1)

            def fn(c, dt=dt, ws=ws, rows=rows, k=k, x=x, xq=xq, y=y):
                check(lib.swamp_quantize_q8_0(x.data_ptr(), pkg.F32, xq.data_ptr(), m * k, s),
                      "swamp_quantize_q8_0")
                check(lib.swamp_qgemm(dt, ws[0].data_ptr(), ws[0].numel(), xq.data_ptr(),
                                      pkg.Q8_0, y.data_ptr(), m, rows, k, s), "swamp_qgemm int8")
            us = timed(fn, reps=10)
            tops = 2 * m * rows * k / us / 1e6
            per.append({"name": name, "dtype": pkg.DTYPE_NAMES[dt], "rows": rows, "k": k,
                        "us": round(us, 1), "TOP/s": round(tops, 1),
                        "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)})
            del ws
        del x, xq, y
    print(json.dumps({"sweep": "llama3-8b prefill int8 MFMA x Q8_0 (quantizer included), "
                               "Q4_K and Q4_0 weights, 2048 tokens", "matrices": per}),
          flush=True)


ROUTE_SHAPES = [("gate_up", 28672, 4096), ("down", 4096, 14336), ("qkv", 6144, 4096),
                ("o_proj", 4096, 4096)]
ROUTE_MS = (256, 512, 1024, 2048)


def stream_reference(torch):
    """torch's own streaming kernels over 1 GiB of fp32 on this device, as a
    reference for what a plain kernel streams from HBM: sum and amax read
    the buffer once, copy reads it and writes another.  Two buffers
    alternate, 3 untimed calls, then the mean of 20 timed with events."""
    n = 1 << 28
    xs = [torch.randn(n, device="cuda") for _ in range(2)]
    dst = torch.empty_like(xs[0])

    def timed(fn, reps=20):
        for i in range(3):
            fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(reps):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / reps

    out = {"stream_ref": "torch kernels over 1 GiB fp32", "bytes_read": 4 * n}
    for name, fn, moved in (("sum", lambda i: xs[i % 2].sum(), 4 * n),
                            ("amax", lambda i: xs[i % 2].amax(), 4 * n),
                            ("copy", lambda i: dst.copy_(xs[i % 2]), 8 * n)):
        t = timed(fn)
        out[name] = {"us": round(t * 1e6, 1), "GB/s": round(moved / t / 1e9, 1),
                     "frac_hbm_peak": round(moved / t / 1e9 / HBM_PEAK_GBS, 4)}
    return out


def gemv_fixed_cost(pkg, torch, stream, lib):
    """Decode GEMV time against row count at fixed K (Q4_0, fp32 x; mean of
    50 launches over rotated weight copies behind a GPU sleep): the
    intercept is the fixed cost of a launch, the slope the streaming rate.
    Beside it, a one-element torch fill timed the same way: the period of
    back-to-back launches of a kernel that does nothing."""
    s = stream.cuda_stream

    def timed(fn, reps=50):
        for i in range(5):
            fn(i)
        torch.cuda.synchronize()
        torch.cuda._sleep(20_000_000)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(reps):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    out = {"gemv_fixed_cost": "swamp_qgemv Q4_0 fp32 x, us and GB/s against rows", "lines": []}
    for k in (4096, 14336):
        pts = []
        for rows in (64, 512, 1024, 2048, 4096, 6144, 8192, 16384, 28672):
            raw = pkg.synth_quantized(pkg.Q4_0, SEED ^ 0xF00 ^ rows, 0.02, rows, k)
            n_cp = max(2, min(16, int(600e6 // raw.size) + 1))
            d0 = torch.from_numpy(raw).cuda()
            ws = [d0] + [d0.clone() for _ in range(n_cp - 1)]
            x = torch.from_numpy(pkg.fill_normal(SEED ^ 0xF01, 1.0, 1, k)[0]).cuda()
            y = torch.empty(rows, dtype=torch.float32, device="cuda")
            us = timed(lambda c: _check(pkg, lib.swamp_qgemv(pkg.Q4_0, ws[c % n_cp].data_ptr(),
                                                             raw.size, x.data_ptr(), y.data_ptr(),
                                                             rows, k, s), "swamp_qgemv"))
            pts.append({"rows": rows, "bytes": int(raw.size), "us": round(us, 2),
                        "GB/s": round(raw.size / us / 1e3, 1)})
            del ws, d0, x, y
        a, b = pts[-2], pts[-1]
        out["lines"].append({"k": k, "points": pts,
                             "slope_GB/s": round((b["bytes"] - a["bytes"]) / (b["us"] - a["us"]) / 1e3, 1)})
    one = torch.empty(1, dtype=torch.float32, device="cuda")
    out["empty_kernel_period_us"] = round(timed(lambda c: one.fill_(1.0)), 2)
    return out


def gemv_stages(pkg, torch, stream, reps=5):
    """Where a decode GEMV launch spends its time: libswamp_gpu_stamps.so
    (libswamp_gpu.so with the decode GEMV's stage stamps compiled in) runs
    each 8B Q4_0 matrix (fp32 x) after 20 warm launches over rotated weight
    copies; every wave records the real-time counter at kernel entry, x
    landed, x fragment built, first tile stored and last tile stored.
    Times are microseconds from the first wave's entry, median over waves
    (and over `reps` launches), with the last wave's end; beside them the
    launch's duration from HIP events (which adds the dispatch before the
    first wave starts and the completion after the last ends)."""
    import ctypes
    import numpy as np
    lib = ctypes.CDLL(os.path.join(REPO, "llamanyon.rs_amd", "libswamp_gpu_stamps.so"))
    lib.swamp_gemv_stage_stamps.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    lib.swamp_qgemv.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    if lib.swamp_gpu_init() != 0:
        raise RuntimeError("swamp_gpu_init failed (stamps library)")
    s = stream.cuda_stream
    n_slots = 16384 * 8
    buf = np.zeros(n_slots, dtype=np.uint64)
    names = ["entry", "x_landed", "xfrag_built", "first_tile_stored", "last_tile_stored"]
    out = {"gemv_stages": "swamp_qgemv Q4_0 fp32 x, us from the first wave's entry", "shapes": []}
    for i, (name, rows, k) in enumerate(DECODE_SHAPES):
        raw = pkg.synth_quantized(pkg.Q4_0, SEED ^ 0x700 ^ i, 0.02, rows, k)
        n_cp = max(2, min(8, int(900e6 // raw.size) + 1))
        d0 = torch.from_numpy(raw).cuda()
        ws = [d0] + [d0.clone() for _ in range(n_cp - 1)]
        x = torch.from_numpy(pkg.fill_normal(SEED ^ 0x701, 1.0, 1, k)[0]).cuda()
        y = torch.empty(rows, dtype=torch.float32, device="cuda")

        def launch(c):
            rc = lib.swamp_qgemv(pkg.Q4_0, ws[c % n_cp].data_ptr(), raw.size, x.data_ptr(),
                                 y.data_ptr(), rows, k, s)
            if rc != 0:
                raise pkg.GpuError(rc, "swamp_qgemv (stamps library)")
        per = {n: [] for n in names[1:]}
        ends, spreads, durs, waves = [], [], [], 0
        for r in range(reps):
            for c in range(20):
                launch(c)
            torch.cuda.synchronize()
            if lib.swamp_gemv_stage_stamps(buf.ctypes.data, 0, 1) != 0:
                raise RuntimeError("swamp_gemv_stage_stamps failed")
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            launch(21 + r)  # keeps the card busy up to the timed launch
            e0.record(stream)
            launch(22 + r)
            e1.record(stream)
            torch.cuda.synchronize()
            durs.append(e0.elapsed_time(e1) * 1e3)
            if lib.swamp_gemv_stage_stamps(buf.ctypes.data, n_slots, 1) != 0:
                raise RuntimeError("swamp_gemv_stage_stamps failed")
            t = buf.reshape(-1, 8)[:, :5].astype(np.int64)
            t = t[(t[:, 0] > 0) & (t[:, 4] > 0)]
            waves = len(t)
            rel = (t - t[:, 0].min()) * 0.01  # 100 MHz counter -> us
            for j, n in enumerate(names[1:], start=1):
                per[n].append(float(np.median(rel[:, j])))
            ends.append(float(rel[:, 4].max()))
            spreads.append(float(rel[:, 0].max()))
        line = {"name": name, "rows": rows, "k": k, "waves": waves,
                "event_us": round(float(np.median(durs)), 2),
                "entry_spread_us": round(float(np.median(spreads)), 2)}
        for n in names[1:]:
            line[n + "_us"] = round(float(np.median(per[n])), 2)
        line["last_wave_end_us"] = round(float(np.median(ends)), 2)
        out["shapes"].append(line)
        del ws, d0, x, y
    return out


def mfma_probe(iters=8000, reps=3):
    """The matrix-core issue microbenchmark (csrc/probe_mfma.hip): one
    workgroup per CU issuing bf16 32x32x16 MFMAs with V VALU fmas per MFMA
    in the same wave (kind 0, one wave per SIMD), in both of two waves per
    SIMD (kind 1) or in a second wave beside an MFMA-only one (kind 2), with
    constant or random operands and with or without a 16-byte LDS fragment
    read per MFMA."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(REPO, "llamanyon.rs_amd", "libswamp_probe.so"))
    kinds = {0: "1 wave/SIMD, VALU in the MFMA wave", 1: "2 waves/SIMD, both MFMA + VALU",
             2: "2 waves/SIMD, MFMA wave + VALU wave"}
    n = lib.swamp_probe_mfma_configs(-1, None, None, None, None)
    rows = []
    for i in range(n):
        kind, valu, rnd, lds = (ctypes.c_int() for _ in range(4))
        lib.swamp_probe_mfma_configs(i, ctypes.byref(kind), ctypes.byref(valu), ctypes.byref(rnd),
                                     ctypes.byref(lds))
        ms, mfmas = ctypes.c_float(), ctypes.c_double()
        if lib.swamp_probe_mfma_run(i, iters, reps, ctypes.byref(ms), ctypes.byref(mfmas)) != 0:
            raise RuntimeError(f"swamp_probe_mfma_run({i}) failed")
        tf = mfmas.value * 32768.0 / (ms.value * 1e-3) / 1e12
        rows.append({"kind": kinds[kind.value], "valu_per_mfma": valu.value,
                     "operands": "random" if rnd.value else "constant",
                     "lds_read_per_mfma": bool(lds.value), "ms": round(ms.value, 3),
                     "TFLOP/s": round(tf, 1), "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)})
    return {"mfma_probe": "V_MFMA_F32_32X32X16_BF16 throughput, one workgroup per CU",
            "configs": rows}


def route_times(pkg, torch, s):
    """us per swamp_qgemm call (Q4_0 weights, bf16 x; mean of 20 after 10
    warm-up calls) for each 8B shape and prompt length, through whichever
    route SWAMP_GEMM_ROUTE forces in this process."""
    import numpy as np
    lib = pkg.gpu_lib()
    out = {}
    for i, (name, rows, k) in enumerate(ROUTE_SHAPES):
        w = torch.from_numpy(pkg.synth_quantized(pkg.Q4_0, SEED ^ 0x300 ^ i, 0.02, rows, k)).cuda()
        for m in ROUTE_MS:
            xb = torch.from_numpy(pkg.to_bf16_bits(pkg.fill_normal(SEED ^ 0x400 ^ m, 1.0, m, k))
                                  .view(np.int16)).cuda()
            y = torch.empty(m, rows, dtype=torch.float32, device="cuda")

            def call():
                rc = lib.swamp_qgemm(pkg.Q4_0, w.data_ptr(), w.numel(), xb.data_ptr(), pkg.BF16,
                                     y.data_ptr(), m, rows, k, s)
                if rc != 0:
                    raise pkg.GpuError(rc, "swamp_qgemm")
            for _ in range(10):
                call()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(20):
                call()
            e1.record()
            torch.cuda.synchronize()
            out[f"{name}@{m}"] = round(e0.elapsed_time(e1) * 1e3 / 20, 1)
    return out


def route_crossover():
    """The prefill GEMM's two routes side by side: each timed in a child
    process with SWAMP_GEMM_ROUTE set (so that neither route's first calls
    share a process with the other's)."""
    import subprocess
    res = {}
    for route in ("fused", "dq"):
        env = dict(os.environ, SWAMP_GEMM_ROUTE=route)
        p = subprocess.run([sys.executable, os.path.abspath(__file__), "--route-times"], env=env,
                           capture_output=True, text=True, timeout=600)
        if p.returncode != 0:
            raise SystemExit(f"route {route}: child failed ({p.returncode}): {p.stderr[-2000:]}")
        res[route] = json.loads([ln for ln in p.stdout.splitlines() if ln.startswith("{")][-1])
    table = []
    for name, rows, k in ROUTE_SHAPES:
        for m in ROUTE_MS:
            key = f"{name}@{m}"
            flop = 2.0 * m * rows * k
            table.append({"name": name, "m": m, "rows": rows, "k": k,
                          "fused_us": res["fused"][key], "dq_us": res["dq"][key],
                          "faster": "dq" if res["dq"][key] < res["fused"][key] else "fused",
                          "best_frac_bf16_peak": round(flop / (min(res["dq"][key],
                                                                   res["fused"][key]) * 1e-6)
                                                       / 1e12 / BF16_PEAK_TFLOPS, 4)})
    print(json.dumps({"route_crossover": "swamp_qgemm Q4_0, bf16 x, 8B shapes; mean of 20 calls "
                                         "after 10 warm-up calls per route",
                      "shapes": table}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--settle", type=float, default=0.3,
                    help="seconds of untimed decode steps before the warm-up steps")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-small-batch", action="store_true",
                    help="leave out the 8B Q4_K small-batch lines and their CPU lines")
    ap.add_argument("--no-70b", action="store_true",
                    help="leave out the 70B decode layer and 4096-token prefill lines")
    ap.add_argument("--cpu-threads", type=str, default="6,max",
                    help="thread counts of the CPU baseline, comma-separated; 'max' is every "
                         "thread of this host's share (the reference's pool size is 6)")
    ap.add_argument("--copies", type=int, default=3, help="weight-set copies rotated per step")
    ap.add_argument("--sweep", action="store_true",
                    help="also print one line per extra workload (more token counts, Q6_K, "
                         "producers, the rest of the 70B prefill, int8 with Q4_K) after the "
                         "main line")
    ap.add_argument("--pmc-batched", type=int, default=0, metavar="N",
                    help="only run 5 swamp_qgemv_batched launches of N tokens on each 8B sweep "
                         "matrix (Q4_K, lm_head Q8_0), for rocprofv3 --pmc counter passes; no JSON")
    ap.add_argument("--pmc-gemm", nargs="?", const="bf16", choices=["bf16", "int8"],
                    help="only run 5 calls of the 2048-token gate+up prefill GEMM (Q4_0 weights; "
                         "x bf16, or int8: x quantized to Q8_0 on the device, then the int8 "
                         "GEMM) and one 256 MiB device copy (for rocprofv3 --pmc), no JSON")
    ap.add_argument("--route-crossover", action="store_true",
                    help="only time swamp_qgemm (Q4_0, bf16 x) at 256..2048 tokens on the 8B "
                         "shapes through each prefill route, forced with SWAMP_GEMM_ROUTE in two "
                         "child processes; one JSON line")
    ap.add_argument("--route-times", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--pmc-decode", action="store_true",
                    help="only run 5 swamp_qgemv launches of each Q4_0 decode matrix (fp32 x) "
                         "over the rotated weight copies, for rocprofv3 --pmc counter passes; "
                         "no JSON")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="only run 5 launches of the dominant kernel and one 256 MiB device copy "
                         "(the calibration for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE), no JSON")
    ap.add_argument("--gemv-fixed-cost", action="store_true",
                    help="only time the decode GEMV (Q4_0) against row count at K = 4096 and "
                         "14336, beside an empty kernel's launch period; one JSON line")
    ap.add_argument("--gemv-stages", action="store_true",
                    help="only time the stages of each 8B decode GEMV launch (stage stamps of "
                         "libswamp_gpu_stamps.so: x landed, first tile, last tile); one JSON line")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="only run the matrix-core issue microbenchmark (libswamp_probe.so): "
                         "bf16 MFMA throughput with VALU work in the same or a second wave per "
                         "SIMD, random or constant operands, LDS fragment reads; one JSON line")
    ap.add_argument("--stream-ref", action="store_true",
                    help="only time torch's own streaming kernels over 1 GiB of fp32 (sum and "
                         "amax: one read; copy: one read and one write) as a reference for the "
                         "decode GEMV's weight stream; one JSON line")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this path has no "
              "multi-GPU code: row-sharding across GPUs is a design note, not a build.",
              file=sys.stderr)
        sys.exit(2)

    if args.route_crossover:
        route_crossover()
        return

    import numpy as np
    import torch

    pkg = _load("llamanyon_rs_amd", os.path.join(REPO, "llamanyon.rs_amd", "__init__.py"))
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a HIP device")
    torch.cuda.set_device(0)
    pkg.init()
    stream = torch.cuda.current_stream()
    s = stream.cuda_stream

    if args.route_times:
        print(json.dumps(route_times(pkg, torch, s)), flush=True)
        return
    if args.mfma_probe:
        print(json.dumps(mfma_probe()), flush=True)
        return
    if args.gemv_stages:
        print(json.dumps(gemv_stages(pkg, torch, stream)), flush=True)
        return
    if args.gemv_fixed_cost:
        print(json.dumps(gemv_fixed_cost(pkg, torch, stream, pkg.gpu_lib())), flush=True)
        return
    if args.stream_ref:
        print(json.dumps(stream_reference(torch)), flush=True)
        return

    # ---- data: one host-quantized weight set, cloned on the device -------
    sets = [[] for _ in range(args.copies)]
    xs, ys = [], []
    for i, (_, rows, k) in enumerate(DECODE_SHAPES):
        raw = pkg.synth_quantized(pkg.Q4_0, SEED ^ i, 0.02, rows, k)
        d0 = torch.from_numpy(raw).cuda()
        sets[0].append(d0)
        for c in range(1, args.copies):
            sets[c].append(d0.clone())
        xs.append(torch.from_numpy(pkg.fill_normal(SEED ^ 0xA11CE ^ i, 1.0, 1, k)[0]).cuda())
        ys.append(torch.empty(rows, dtype=torch.float32, device="cuda"))
    step_bytes = sum(alg_bytes_gemv(18, r, k) for _, r, k in DECODE_SHAPES)
    rotated = sum(t.numel() for st in sets for t in st)
    lib = pkg.gpu_lib()

    if args.pmc_gemm:
        # the prefill GEMM under rocprofv3 --pmc: 5 calls of the 2048-token
        # gate+up (each a full-tile and a half-tile launch), then the same
        # calibration copy as --pmc-probe
        name, rows, k = PREFILL_SHAPES[0]
        pm = PREFILL_MS[0]
        raw = pkg.synth_quantized(pkg.Q4_0, SEED ^ 0x100, 0.02, rows, k)
        w = torch.from_numpy(raw).cuda()
        xf = pkg.fill_normal(SEED ^ 0x200, 1.0, pm, k)
        yg = torch.empty((pm, rows), dtype=torch.float32, device="cuda")
        if args.pmc_gemm == "int8":
            xd = torch.from_numpy(xf).cuda()
            xg = torch.empty(pm * k // 32 * 34, dtype=torch.uint8, device="cuda")
        else:
            xg = torch.from_numpy(pkg.to_bf16_bits(xf).view(np.int16)).cuda()
        for _ in range(5):
            if args.pmc_gemm == "int8":
                rc = lib.swamp_quantize_q8_0(xd.data_ptr(), pkg.F32, xg.data_ptr(), pm * k, s)
                if rc == 0:
                    rc = lib.swamp_qgemm(pkg.Q4_0, w.data_ptr(), w.numel(), xg.data_ptr(),
                                         pkg.Q8_0, yg.data_ptr(), pm, rows, k, s)
            else:
                rc = lib.swamp_qgemm(pkg.Q4_0, w.data_ptr(), w.numel(), xg.data_ptr(), pkg.BF16,
                                     yg.data_ptr(), pm, rows, k, s)
            if rc != 0:
                raise pkg.GpuError(rc, "swamp_qgemm")
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"pmc gemm: 5 x swamp_qgemm Q4_0 {name} {pm}x{rows}x{k} ({args.pmc_gemm} x), then a "
              f"{src.numel()}-byte device copy", flush=True)
        return

    if args.pmc_batched:
        # the small batch under rocprofv3 --pmc: 5 launches per 8B matrix,
        # in sweep order, each matrix with its own weights and activations
        n_tok = args.pmc_batched
        for i, (name, rows, k) in enumerate(SWEEP_8B):
            dt = pkg.Q8_0 if name == "lm_head" else pkg.Q4_K
            w = torch.from_numpy(pkg.synth_quantized(dt, SEED ^ 0x300 ^ i, 0.02, rows, k)).cuda()
            x = torch.from_numpy(pkg.fill_normal(SEED ^ 0x400 ^ i, 1.0, n_tok, k)).cuda()
            y = torch.empty((n_tok, rows), dtype=torch.float32, device="cuda")
            for _ in range(5):
                rc = lib.swamp_qgemv_batched(dt, w.data_ptr(), w.numel(), x.data_ptr(), y.data_ptr(),
                                             n_tok, rows, k, 0, s)
                if rc != 0:
                    raise pkg.GpuError(rc, "swamp_qgemv_batched")
            torch.cuda.synchronize()
            print(f"pmc batched: 5 x swamp_qgemv_batched {name} {rows}x{k} n_tok {n_tok}", flush=True)
            del w, x, y
        return

    if args.pmc_decode:
        # the decode step's matrices under rocprofv3 --pmc: 5 launches of each
        # (over the rotated weight copies), matrix after matrix, nothing else
        for i, (name, rows, k) in enumerate(DECODE_SHAPES):
            for it in range(5):
                w = sets[it % args.copies][i]
                rc = lib.swamp_qgemv(pkg.Q4_0, w.data_ptr(), w.numel(), xs[i].data_ptr(),
                                     ys[i].data_ptr(), rows, k, s)
                if rc != 0:
                    raise pkg.GpuError(rc, "swamp_qgemv")
            torch.cuda.synchronize()
            print(f"pmc decode: 5 x swamp_qgemv Q4_0 {name} {rows}x{k}", flush=True)
        return

    if args.pmc_probe:
        # HBM traffic of the dominant kernel under rocprofv3 --pmc: its
        # launches (one per weight copy), then a plain copy of known size
        # whose counter reading calibrates the counter (bytes per unit).
        i = max(range(len(DECODE_SHAPES)), key=lambda j: DECODE_SHAPES[j][1] * DECODE_SHAPES[j][2])
        _, rows, k = DECODE_SHAPES[i]
        for it in range(5):
            w = sets[it % args.copies][i]
            rc = lib.swamp_qgemv(pkg.Q4_0, w.data_ptr(), w.numel(), xs[i].data_ptr(),
                                 ys[i].data_ptr(), rows, k, s)
            if rc != 0:
                raise pkg.GpuError(rc, "swamp_qgemv")
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"pmc probe: 5 x swamp_qgemv Q4_0 {rows}x{k} "
              f"({alg_bytes_gemv(18, rows, k)} algorithmic bytes each), then a "
              f"{src.numel()}-byte device copy", flush=True)
        return

    def launch(c, i, fn=lib.swamp_qgemv):
        _, rows, k = DECODE_SHAPES[i]
        w = sets[c][i]
        rc = fn(pkg.Q4_0, w.data_ptr(), w.numel(), xs[i].data_ptr(), ys[i].data_ptr(), rows, k, s)
        if rc != 0:
            raise pkg.GpuError(rc, "swamp_qgemv")

    def settle(fn=lib.swamp_qgemv):
        # Untimed steps for args.settle seconds before the warm-up steps: under
        # sustained load the card takes some milliseconds to reach the clock it
        # then holds (the first 50 steps after a pause run up to 20% slower).
        t_end = time.perf_counter() + args.settle
        it = 0
        while time.perf_counter() < t_end:
            for _ in range(20):
                for i in range(len(DECODE_SHAPES)):
                    launch(it % args.copies, i, fn)
                it += 1
            torch.cuda.synchronize()

    settle()
    for it in range(args.warmup):
        for i in range(len(DECODE_SHAPES)):
            launch(it % args.copies, i)
    torch.cuda.synchronize()

    # ---- timed region: exactly K steps ------------------------------------
    n = len(DECODE_SHAPES)
    dom = max(range(n), key=lambda i: DECODE_SHAPES[i][1] * DECODE_SHAPES[i][2])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for it in range(args.steps):
        for i in range(n):
            launch(it % args.copies, i)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # ---- the dominant kernel's launch duration ------------------------------
    # The lm_head GEMV (70% of the step's bytes) alone: 10 bursts of 20
    # back-to-back launches over the rotated weight copies, each burst
    # between two HIP timing events on the launch stream and queued behind a
    # GPU sleep, so the launches follow each other as in the step.  A burst's
    # time over 20 is the kernel's duration plus the gap between two
    # dependent kernels (under 1 us).  An event pair around every single
    # launch would add its own dispatch and completion latency to each one
    # (about 4 us here), so it is not used.
    n_bursts, per_burst = 10, 20
    ev = [(TimingEvent(), TimingEvent()) for _ in range(n_bursts)]
    for b in range(n_bursts):
        torch.cuda.synchronize()
        torch.cuda._sleep(5_000_000)
        ev[b][0].record(s)
        for it in range(per_burst):
            launch((b * per_burst + it) % args.copies, dom)
        ev[b][1].record(s)
    torch.cuda.synchronize()

    dom_name, dom_rows, dom_k = DECODE_SHAPES[dom]
    dom_bytes = alg_bytes_gemv(18, dom_rows, dom_k)
    dom_lat = np.array([a.elapsed_ms(b) for a, b in ev]) * 1e3 / per_burst
    dom_us = float(np.mean(dom_lat))
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    traffic = traffic_from_profiles()
    roofline = {"bound": "hbm", "kernel": f"gemv_kernel<Q4_0> on {dom_name} "
                                          f"{dom_rows}x{dom_k}",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": traffic, "alg_bytes_per_launch": dom_bytes,
                "avg_launch_us": round(dom_us, 2),
                "burst_launch_us_p10_p50_p90": [round(float(v), 2)
                                          for v in np.percentile(dom_lat, [10, 50, 90])]}

    # ---- per-matrix kernel times (outside the timed region) --------------
    # Each matrix alone, 20 back-to-back launches over the rotated copies,
    # queued behind a GPU sleep so the host never starves the GPU.
    def per_matrix(fn):
        out = []
        for i, (name, rows, k) in enumerate(DECODE_SHAPES):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            torch.cuda._sleep(20_000_000)
            e0.record(stream)
            for it in range(20):
                launch(it % args.copies, i, fn)
            e1.record(stream)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / 20
            b = alg_bytes_gemv(18, rows, k)
            out.append({"name": name, "rows": rows, "k": k, "bytes": b, "us": round(us, 2),
                        "GB/s": round(b / (us * 1e-6) / 1e9, 1),
                        "frac_hbm_peak": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        return out

    shapes = per_matrix(lib.swamp_qgemv)

    # ---- the same step on swamp_qgemv_f16x (x rounded to fp16 inside the
    # kernel): a separately labelled line, not the headline
    settle(lib.swamp_qgemv_f16x)
    for it in range(args.warmup):
        for i in range(n):
            launch(it % args.copies, i, lib.swamp_qgemv_f16x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for it in range(args.steps):
        for i in range(n):
            launch(it % args.copies, i, lib.swamp_qgemv_f16x)
    torch.cuda.synchronize()
    ms16 = (time.perf_counter() - t0) * 1e3 / args.steps
    f16x = {"entry": "swamp_qgemv_f16x", "dtype": "q4_0 x f16 -> f32",
            "note": "x rounded to fp16 per 64-weight run inside the kernel; not the reference's "
                    "arithmetic",
            "value": round(step_bytes / (ms16 * 1e-3) / 1e9, 1), "unit": "GB/s",
            "ms_per_step": round(ms16, 4),
            "frac_hbm_peak": round(step_bytes / (ms16 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "shapes": per_matrix(lib.swamp_qgemv_f16x)}

    # ---- prefill GEMM, 2048 and 512 tokens, bf16 / Q8_0 activations ----------
    prefill = None
    if not args.no_prefill:
        prefill = []
        for pm in PREFILL_MS:
            for i, (name, rows, k) in enumerate(PREFILL_SHAPES):
                raw = pkg.synth_quantized(pkg.Q4_0, SEED ^ 0x100 ^ i, 0.02, rows, k)
                w = torch.from_numpy(raw).cuda()
                xf = pkg.fill_normal(SEED ^ 0x200 ^ i, 1.0, pm, k)
                xb = pkg.to_bf16_bits(xf)
                x = torch.from_numpy(xb.view(np.int16)).cuda()
                # int8 variant: the same activations quantized per 32-block to
                # Q8_0 on the device (the quantizer is timed with the GEMM)
                xf_d = torch.from_numpy(xf).cuda()
                xq = torch.empty(pm * k // 32 * 34, dtype=torch.uint8, device="cuda")
                y = torch.empty((pm, rows), dtype=torch.float32, device="cuda")

                def g_bf16():
                    rc = lib.swamp_qgemm(pkg.Q4_0, w.data_ptr(), w.numel(), x.data_ptr(),
                                         pkg.BF16, y.data_ptr(), pm, rows, k, s)
                    if rc != 0:
                        raise pkg.GpuError(rc, "swamp_qgemm")

                def g_int8():
                    rc = lib.swamp_quantize_q8_0(xf_d.data_ptr(), pkg.F32, xq.data_ptr(),
                                                 pm * k, s)
                    if rc == 0:
                        rc = lib.swamp_qgemm(pkg.Q4_0, w.data_ptr(), w.numel(), xq.data_ptr(),
                                             pkg.Q8_0, y.data_ptr(), pm, rows, k, s)
                    if rc != 0:
                        raise pkg.GpuError(rc, "swamp_qgemm int8")

                for xname, g, peak in (("bf16", g_bf16, BF16_PEAK_TFLOPS),
                                       ("q8_0 (int8 MFMA)", g_int8, INT8_PEAK_TOPS)):
                    # 10 untimed calls bring the shader clock to its sustained
                    # level under this load, then the mean of 20 back-to-back
                    for _ in range(10):
                        g()
                    reps = 20
                    e0, e1 = (torch.cuda.Event(enable_timing=True),
                              torch.cuda.Event(enable_timing=True))
                    e0.record(stream)
                    for _ in range(reps):
                        g()
                    e1.record(stream)
                    torch.cuda.synchronize()
                    us = e0.elapsed_time(e1) * 1e3 / reps
                    tops = 2.0 * pm * rows * k / (us * 1e-6) / 1e12
                    prefill.append({"name": name, "m": pm, "rows": rows, "k": k, "x": xname,
                                    "route": gemm_route(torch, False, pm, rows, k, xname),
                                    "us": round(us, 1), "TFLOP/s": round(tops, 1),
                                    "frac_peak": round(tops / peak, 4),
                                    "peak": peak})
                del w, x, y, xf_d, xq

    # ---- 8B Q4_K small batch (lm_head Q8_0) at 1, 4, 8, 16 tokens; 70B Q4_K
    # decode layer (lm_head Q8_0) and 4096-token bf16 prefill --------------------
    small = None
    if not args.no_small_batch:
        small = {"workload": "llama3-8b Q4_K qkv 6144x4096, o_proj 4096x4096, gate_up "
                             "28672x4096, down 4096x14336 + lm_head 128256x4096 Q8_0; "
                             "W ~ N(0,0.02), x ~ N(0,1) fp32; each matrix timed alone "
                             "(mean of 20 launches over rotated weight copies), summed",
                 "lines": layer_lines(pkg, torch, stream, lib, SWEEP_8B, 0.02, (1, 4, 8, 16),
                                      SEED)}
    dec70 = pre70 = None
    if not args.no_70b:
        dec70 = {"workload": "llama3-70b Q4_K qkv 10240x8192, o_proj 8192x8192, gate_up "
                             "57344x8192, down 8192x28672 + lm_head 128256x8192 Q8_0, batch 1; "
                             "W ~ N(0,0.015), x ~ N(0,1) fp32; each matrix timed alone, summed",
                 **layer_lines(pkg, torch, stream, lib, SWEEP_70B, 0.015, (1,), SEED ^ 0x70B)[0]}
        pre70 = prefill_70b_lines(pkg, torch, np, stream, lib, ("gate_up", "down", "qkv"))

    tcounts = []
    for t in args.cpu_threads.split(","):
        n_t = cpu_threads_available() if t.strip() == "max" else int(t)
        if n_t not in tcounts:
            tcounts.append(n_t)
    cpu = None if args.no_cpu else cpu_baseline(pkg, tcounts)
    if small is not None and not args.no_cpu:
        small["cpu"] = cpu_small_batch(pkg, tcounts)

    out = {
        "metric": "decode Q4 GEMV HBM GB/s (% peak) at 8B shapes; prefill GEMM TOPS @2048 tok",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x f32 -> f32",
        "data": "synthetic (W ~ N(0,0.02) quantized to Q4_0 on the host, x ~ N(0,1) fp32)",
        "config": {"workload": "llama3-8b decode layer sweep, Q4_0, batch 1: qkv 6144x4096, "
                               "o_proj 4096x4096, gate_up 28672x4096, down 4096x14336, "
                               "lm_head 128256x4096",
                   "step_alg_bytes": step_bytes, "weight_copies_rotated": args.copies,
                   "rotated_weight_bytes": rotated, "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "shapes": shapes,
        "decode_f16x": f16x,
        "prefill": prefill,
        "small_batch": small,
        "decode_70b": dec70,
        "prefill_70b": pre70,
    }
    print(json.dumps(out), flush=True)
    if args.sweep:
        run_sweep(pkg, torch, np, stream, lib)
        if not args.no_cpu:
            cpu_sweep(pkg, tcounts)


if __name__ == "__main__":
    main()
