"""CPU-side checks of the drop-in boundary: the HIP library loads (no GPU
needed), exports exactly what include/lbt.h declares, the ctypes binding
covers every declaration, and with no GPU present entry points fail with a
status code instead of aborting."""
import ctypes as C
import re
from pathlib import Path

import pytest

import lbt_hip

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "lbt.h"


def declared() -> set:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(lbt_\w+)\s*\(", text))


def test_library_exports_every_declaration():
    lib = lbt_hip.load_library()
    for name in declared():
        assert hasattr(lib, name), name


def test_binding_matches_header():
    assert set(lbt_hip.SIGNATURES) == declared()


def test_no_gpu_returns_status():
    import os

    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    lib = lbt_hip.load_library()
    h = C.c_void_p()
    assert lib.lbt_ctx_create(0, C.byref(h)) != 0
    assert lib.lbt_version().decode().startswith("lbt-hip")


def test_null_arguments_are_errors_not_crashes():
    """Entry points reject null handles with a status (the reference asserts;
    the C ABI never aborts).  Runs without a GPU."""
    lib = lbt_hip.load_library()
    out = C.c_void_p()
    assert lib.lbt_q8head_from_bf16(None, None, C.byref(out)) != 0
    assert lib.lbt_q8head_linear(None, None, None, 1, None) != 0
    assert lib.lbt_q8head_linear_dev(None, None, None, 1, None) != 0
    assert lib.lbt_q8head_read(None, None, None, None) != 0
    assert lib.lbt_model_set_head(None, 1) != 0
    assert lib.lbt_bf16_linear(None, None, None, 1, None) != 0
    assert lib.lbt_gemm_i32(None, None, None, None, 1, None) != 0
    lib.lbt_q8head_free(None)
    lib.lbt_bf16_free(None)
    assert lib.lbt_sched_new(None, 2, 16, C.byref(out)) != 0
    assert lib.lbt_sched_step(None, None) != 0
    assert lib.lbt_sched_result(None, 1, None, 0, None, None) != 0
    assert lib.lbt_batch_reset(None, 0) != 0
    assert lib.lbt_sched_release(None, 1) != 0
    lib.lbt_sched_free(None)


def test_header_compiles_as_c():
    import subprocess

    src = '#include "lbt.h"\nint main(void){lbt_config c; (void)c; return 0;}\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{REPO / 'include'}", "-x", "c", "-", "-o",
                        "/dev/null"], input=src, text=True, capture_output=True)
    assert r.returncode == 0, r.stderr
