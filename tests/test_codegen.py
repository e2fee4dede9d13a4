"""Code-generation checks of the decode GEMV (CPU only: hipcc cross-compiles
for gfx950).

The item kernel stages x in LDS by direct-to-LDS DMA and then waits with a
hand-counted s_waitcnt vmcnt(N): the memory counter is in order, so N must
equal the number of vector-memory loads issued after the last DMA (the first
tile's weight loads).  If the compiler ever issued another vector load in
between, or turned one into a scalar load, the wait would release before the
last DMA landed and a workgroup would read stale LDS -- wrong results that
depend on timing.  This test compiles the two translation units to assembly
and checks N against the loads actually emitted, for every instantiation."""
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


def _kernels(lines):
    cur, body = None, []
    for line in lines:
        m = re.match(r"^(_ZN12_GLOBAL__N_111gemv_kernel\w+):", line)
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


def test_staged_x_wait_counts_match_emitted_loads(tmp_path):
    tus = ["gemv.hip", "gemv_fused.hip"]
    with ThreadPoolExecutor(2) as ex:
        asms = list(ex.map(lambda t: _asm(t, str(tmp_path / (t + ".s"))), tus))
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
