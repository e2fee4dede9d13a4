"""Code-generation checks of the decode GEMV (CPU only: hipcc cross-compiles
for gfx950).

The item kernel stages x in LDS by direct-to-LDS DMA and then waits with a
hand-counted s_waitcnt vmcnt(N): the memory counter is in order, so N must
equal the number of vector-memory loads issued after the last DMA (the first
tile's weight loads).  If the compiler ever issued another vector load in
between, or turned one into a scalar load, the wait would release before the
last DMA landed and a workgroup would read stale LDS -- wrong results that
depend on timing.  This test compiles the two translation units to assembly
and checks N against the loads actually emitted, for every instantiation.
The same assembly shows whether any kernel spills registers to scratch."""
import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "llamanyon.rs_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")


def _asm(tu, out):
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-I" + os.path.join(REPO, "include"),
           "-I" + CSRC, "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "--cuda-device-only", "-S", os.path.join(CSRC, tu), "-o", out]
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    with open(out) as f:
        return f.read().split("\n")


def _kernels(lines, name=r"11gemv_kernel"):
    cur, body = None, []
    for line in lines:
        m = re.match(r"^(_ZN12_GLOBAL__N_1" + name + r"\w+):", line)
        if m:
            cur, body = m.group(1), []
            continue
        if cur is not None:
            body.append(line)
            if "s_endpgm" in line:
                yield cur, body
                cur = None


def _staged_wait(body):
    """(N of the first 'vmcnt(N); s_barrier', vector loads between the last
    LDS DMA before it and the wait), or None for kernels without staging."""
    for i in range(1, len(body)):
        if "s_barrier" in body[i] and "vmcnt(" in body[i - 1]:
            n = int(re.search(r"vmcnt\((\d+)\)", body[i - 1]).group(1))
            dma = [j for j in range(i) if body[j].rstrip().endswith(" lds")]
            if not dma:
                return None
            loads = sum(1 for j in range(dma[-1] + 1, i)
                        if re.search(r"\b(buffer_load|global_load|flat_load)", body[j]))
            return n, loads
    return None


_VMEM = re.compile(r"\b(buffer_load|global_load|flat_load)")


def _gemm_kernels(lines):
    cur, body = None, []
    for line in lines:
        m = re.match(r"^(_ZN12_GLOBAL__N_116gemm_bf16_kernel\w+):", line)
        if m:
            cur, body = m.group(1), []
            continue
        if cur is not None:
            body.append(line)
            if "s_endpgm" in line:
                yield cur, body
                cur = None


def _gemm_wait_problems(body):
    """Checks the prefill GEMM's hand-counted waits.  The prologue issues
    four activation DMA groups and two weight items in the order x0 x1 x2
    w0 x3 w1 and then waits with vmcnt(N): N must be the number of loads
    after x1, i.e. 2 P with P = loads per K step.  Each K step of the main
    loop (two per trip, four for Q4_K) issues P loads and closes with vmcnt(2 P) +
    s_barrier, which leaves exactly the previous and the current step's
    loads in flight.  (The odd last step after the loop may issue fewer:
    its weight prefetch is dead and removed.)"""
    bars = [i for i, l in enumerate(body) if l.strip().startswith("s_barrier")]

    def wait_before(b):
        for j in range(b - 1, max(b - 4, -1), -1):
            m = re.search(r"vmcnt\((\d+)\)", body[j])
            if m:
                return int(m.group(1))
        return None

    probs = []
    pro = [l for l in body[:bars[0]] if _VMEM.search(l)]
    dmas = [l for l in pro if l.rstrip().endswith(" lds")]
    k_dma = len(dmas) // 4
    p = (len(pro) - 2 * k_dma) // 2
    if len(dmas) != 4 * k_dma or not all(l.rstrip().endswith(" lds") for l in pro[:2 * k_dma]):
        probs.append("prologue does not start with two DMA groups")
    if wait_before(bars[0]) != 2 * p:
        probs.append("prologue wait %s != %d" % (wait_before(bars[0]), 2 * p))
    head = [i for i, l in enumerate(body) if "Loop Header" in l]
    if not head:
        return probs + ["no K loop found"]
    label = body[head[0]].split(":")[0]
    back = [i for i, l in enumerate(body)
            if re.match(r"\s+s_(c)?branch", l) and re.search(re.escape(label) + r"\b", l)]
    if not back:
        return probs + ["no K loop back-branch"]
    lo, hi = head[0], back[-1]
    loop_bars = [b for b in bars if lo < b < hi]
    if len(loop_bars) not in (2, 4):  # two steps per trip (four for Q4_K)
        probs.append("%d barriers in the K loop, expected 2 or 4" % len(loop_bars))
    prev = lo
    for b in loop_bars:
        loads = sum(1 for l in body[prev:b] if _VMEM.search(l))
        n = wait_before(b)
        if loads != p or n != 2 * p:
            probs.append("step with %d loads waits vmcnt(%s), expected %d / %d" % (loads, n, p, 2 * p))
        prev = b
    # no full drain inside the K loop, no scratch traffic anywhere
    if any("vmcnt(0)" in l for l in body[lo:hi + 1]):
        probs.append("vmcnt(0) inside the K loop")
    if any("scratch_" in l for l in body):
        probs.append("scratch memory access")
    return probs


_TUS = ["api.hip", "device.hip", "dequant.hip", "gemv.hip", "gemv_fused.hip", "gemv_tokens.hip",
        "gemv_batched.hip",
        "gemm.hip", "gemm_dq.hip", "gemm_bb.hip",
        "gemm_i8.hip", "gguf.hip", "producers.hip"]


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    """Device assembly of every translation unit of the library, by name."""
    d = tmp_path_factory.mktemp("asm")
    with ThreadPoolExecutor(4) as ex:
        return dict(zip(_TUS, ex.map(lambda t: _asm(t, str(d / (t + ".s"))), _TUS)))


def test_no_kernel_uses_scratch(asm):
    """Register spills go to scratch memory (per-lane HBM traffic on the hot
    loops).  Every kernel of the library must fit its registers: the small
    batch runs 16 waves per CU (128 VGPRs each), the GEMV up to 2 items per
    lane."""
    checked, bad = 0, []
    for tu, lines in asm.items():
        name = None
        for line in lines:
            m = re.match(r"^(_Z\w+):", line)
            if m:
                name = m.group(1)
            m = re.match(r"^; ScratchSize: (\d+)", line)
            if m and name:
                checked += 1
                if int(m.group(1)):
                    bad.append((tu, name, int(m.group(1))))
    assert checked >= 300, checked
    assert not bad, bad


def test_gemm_wait_counts_match_emitted_loads(asm):
    lines = asm["gemm.hip"]
    kernels = list(_gemm_kernels(lines))
    # three weight formats x (full, half, quarter tile)
    assert len(kernels) == 9, [k for k, _ in kernels]
    bad = [(name, p) for name, body in kernels for p in [_gemm_wait_problems(body)] if p]
    assert not bad, bad


def _bb_wait_problems(body):
    """Checks the plain bf16 GEMM's hand-counted waits (gemm_bb.hip).  The
    prologue issues three steps of P activation/weight DMAs and waits with
    vmcnt(2 P) (the first step landed).  Each trip of the K loop is one
    step: it issues P DMAs, D of them before its one barrier, and the wait
    before that barrier must be P + D (the previous step's DMAs and this
    step's first D stay in flight: the step after the current one has
    landed).  No other vector-memory access may sit in the loop (a flat
    access to LDS would also count), and no vmcnt(0)."""
    bars = [i for i, l in enumerate(body) if l.strip().startswith("s_barrier")]

    def wait_before(b):
        for j in range(b - 1, max(b - 4, -1), -1):
            m = re.search(r"vmcnt\((\d+)\)", body[j])
            if m:
                return int(m.group(1))
        return None

    probs = []
    pro = [l for l in body[:bars[0]] if _VMEM.search(l)]
    if not pro or not all(l.rstrip().endswith(" lds") for l in pro) or len(pro) % 3:
        return ["prologue is not three steps of DMAs: %d loads" % len(pro)]
    p = len(pro) // 3
    if wait_before(bars[0]) != 2 * p:
        probs.append("prologue wait %s != %d" % (wait_before(bars[0]), 2 * p))
    head = [i for i, l in enumerate(body) if "Loop Header" in l]
    if not head:
        return probs + ["no K loop found"]
    label = body[head[0]].split(":")[0]
    back = [i for i, l in enumerate(body)
            if re.match(r"\s+s_(c)?branch", l) and re.search(re.escape(label) + r"\b", l)]
    if not back:
        return probs + ["no K loop back-branch"]
    lo, hi = head[0], back[-1]
    loop_bars = [b for b in bars if lo < b < hi]
    if len(loop_bars) != 1:
        return probs + ["%d barriers in the K loop, expected 1" % len(loop_bars)]
    mem = [i for i in range(lo, hi + 1) if re.search(r"\b(buffer_|global_|flat_)", body[i])]
    if any(not body[i].rstrip().endswith(" lds") for i in mem):
        probs.append("a vector-memory access other than a DMA in the K loop")
    if len(mem) != p:
        probs.append("%d DMAs in the K loop, expected %d" % (len(mem), p))
    d = sum(1 for i in mem if i < loop_bars[0])
    if wait_before(loop_bars[0]) != p + d:
        probs.append("loop wait %s != %d + %d" % (wait_before(loop_bars[0]), p, d))
    if any("vmcnt(0)" in l for l in body[lo:hi + 1]):
        probs.append("vmcnt(0) inside the K loop")
    return probs


def test_bb_gemm_wait_counts_match_emitted_loads(asm):
    lines = asm["gemm_bb.hip"]
    kernels = list(_kernels(lines, r"14gemm_bb_kernel"))
    # full, 192-row, 128-row and half tiles
    assert len(kernels) == 4, [k for k, _ in kernels]
    bad = [(name, p) for name, body in kernels for p in [_bb_wait_problems(body)] if p]
    assert not bad, bad


def test_staged_x_wait_counts_match_emitted_loads(asm):
    tus = ["gemv.hip", "gemv_fused.hip"]
    asms = [asm[t] for t in tus]
    checked, bad = 0, []
    for tu, lines in zip(tus, asms):
        for name, body in _kernels(lines):
            w = _staged_wait(body)
            if w is None:
                continue
            checked += 1
            if w[0] != w[1]:
                bad.append((tu, name, w))
    # every one-item-per-lane instantiation stages x: plain, RMSNorm, SwiGLU
    assert checked >= 250, checked
    assert not bad, bad[:5]


def test_two_token_gemv_wait_counts_match_emitted_loads(asm):
    """The two-token GEMV waits for its x DMA by counting the first tile's
    loads issued after it: that count must be the loads emitted, in every
    instantiation (4 dtypes x rows per tile x waves per row)."""
    checked, bad = 0, []
    for name, body in _kernels(asm["gemv_tokens.hip"], r"15gemv_tok_kernel"):
        w = _staged_wait(body)
        assert w is not None, name
        checked += 1
        if w[0] != w[1]:
            bad.append((name, w))
    assert checked >= 28, checked
    assert not bad, bad[:5]
