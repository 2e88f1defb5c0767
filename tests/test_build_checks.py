"""Build-time checks of kernels that issue loads the compiler does not track
(inline-asm loads waited for with explicit counts): the compiler does not
know such a register is written late, so a spill, reload or copy of a
pending register would read stale data silently.  The kernels' AMD ISA
(hipcc -S, gfx950) must therefore hold no scratch access while those loads
are in flight: none at all in the LM-head kernels, none between the first
and the last matrix instruction of the GEMM main loops (their epilogues, past
the final wait, may spill).  Runs hipcc on the CPU; no GPU needed."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
CSRC = REPO / "lemonade-burn_amd" / "csrc"
HIPCC = "/opt/rocm/bin/hipcc"

# source file -> (mangled kernel name prefix, region checked)
KERNELS = {
    "decode_ops.hip": [("_ZN3lbt18lmhead_mfma_kernel", "all"), ("_ZN3lbt13lmhead_kernel", "all"), ("_ZN3lbt20lmhead_stream_kernel", "all"),
                       ("_ZN3lbt13q8head_kernel", "all")],
    "ternary_mfma.hip": [("_ZN3lbt13tgemm2_kernel", "mfma"), ("_ZN3lbt13tgemm3_kernel", "mfma")],
}
SCRATCH = re.compile(r"^\s*(scratch_(load|store)|buffer_(load|store)\S*\s.*s\[0:3\])")


def kernel_bodies(src: str) -> dict:
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", f"-I{REPO / 'include'}", "--cuda-device-only", "-S", "-o", "-",
           str(CSRC / src)]
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-2000:]
    bodies, cur = {}, None
    for ln in out.stdout.splitlines():
        m = re.match(r"^(_Z\w+):", ln)
        if m:
            cur = m.group(1)
            bodies[cur] = []
            continue
        if cur and ln.startswith(".Lfunc_end"):
            cur = None
        elif cur:
            bodies[cur].append(ln)
    return bodies


@pytest.mark.skipif(shutil.which(HIPCC) is None, reason="hipcc not installed")
@pytest.mark.parametrize("src", sorted(KERNELS))
def test_no_scratch_while_untracked_loads_are_pending(src):
    bodies = kernel_bodies(src)
    for prefix, region in KERNELS[src]:
        names = [k for k in bodies if k.startswith(prefix)]
        assert names, f"{prefix} not found in {src}"
        for k in names:
            lines = bodies[k]
            if region == "mfma":
                idx = [i for i, ln in enumerate(lines) if "v_mfma" in ln]
                assert idx, k
                lines = lines[idx[0]: idx[-1] + 1]
            bad = [ln.strip() for ln in lines if SCRATCH.match(ln)]
            assert not bad, (k, bad[:4])
