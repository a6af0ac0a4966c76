"""Spill gate: every kernel of the shipped library is compiled (device code
only, the build's own hipcc flags) with the compiler's kernel resource report,
and none may use scratch memory.

A spilled register is reloaded through scratch with a vmcnt wait that also
waits for every global load the wave has in flight, which stalls the
streaming producers of the GEMM and convolution kernels for a whole memory
round trip. Runs on the CPU: hipcc cross-compiles gfx950 without a GPU.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import subprocess
import tempfile

import pytest

from ml_framework_amd import build as hip_build

HIP_FILES = [s for s in hip_build.HIP_SOURCES if s.endswith(".hip")]

# The kernels whose per-lane scratch used to be nonzero, plus the hot kernel of
# every benchmark workload: each must appear in the report (a rename would
# otherwise let the gate pass without looking at them).
MUST_SEE = [
    "fused_bwd_kernel",
    "igemm_ws2_kernel",
    "igemm_ws1_kernel",
    "igemm_ws_kernel",
    "igemm_pipe_kernel",
    "stream_conv_kernel",
    "stream_wgrad_kernel",
    "phase2_conv_kernel",
    "stride2_conv_kernel",
    "wgrad_s2_kernel",
]

_NAME = re.compile(r"remark: Function Name: (\S+)")
_FIELD = re.compile(r"remark:\s+(ScratchSize \[bytes/lane\]|VGPRs Spill|VGPRs|AGPRs): (\d+)")


def _report(src: str, outdir: str) -> list[tuple[str, dict]]:
    flags = [f for f in hip_build.HIP_FLAGS if f != "-Wall"]
    cmd = [hip_build.HIPCC, *flags, "-x", "hip", "--offload-device-only", "-c",
           os.path.join(hip_build.CSRC, src), "-o", os.path.join(outdir, src + ".o"),
           "-Rpass-analysis=kernel-resource-usage"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, f"{src} failed to compile:\n{proc.stderr[-4000:]}"
    kernels: list[tuple[str, dict]] = []
    for line in proc.stderr.splitlines():
        m = _NAME.search(line)
        if m:
            kernels.append((m.group(1), {}))
            continue
        m = _FIELD.search(line)
        if m and kernels:
            kernels[-1][1][m.group(1)] = int(m.group(2))
    return kernels


@pytest.mark.skipif(not os.path.exists(hip_build.HIPCC), reason="hipcc not installed")
def test_no_kernel_uses_scratch():
    with tempfile.TemporaryDirectory() as tmp:
        with cf.ThreadPoolExecutor(min(8, os.cpu_count() or 4)) as ex:
            reports = dict(zip(HIP_FILES, ex.map(lambda s: _report(s, tmp), HIP_FILES)))
    seen = [name for rows in reports.values() for name, _ in rows]
    assert len(seen) > 50, "the resource report listed too few kernels"
    for k in MUST_SEE:
        assert any(k in n for n in seen), f"no kernel named like {k} in the report"
    bad = [(src, name, fields) for src, rows in reports.items() for name, fields in rows
           if fields.get("ScratchSize [bytes/lane]", 0) != 0 or fields.get("VGPRs Spill", 0) != 0]
    assert not bad, "kernels using scratch:\n" + "\n".join(
        f"  {src}: {name} {fields}" for src, name, fields in bad)
