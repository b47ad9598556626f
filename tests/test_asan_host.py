"""The C ABI's host code under AddressSanitizer (CPU only, no GPU).

Every source of the library is compiled with the host side instrumented
(`-Xarch_host -fsanitize=address`; the device code is built as usual) and
linked with `tests/asan/fk_abi_asan.cpp`, which calls every entry point of
`include/fastkernels_hip.h` with arguments the host-side validation must
refuse before any HIP call (NULL pointers, sizes out of range, misaligned
pointers, short workspaces), and the size and status functions over edge
inputs.  ASan stops the run at the first memory error in the validation,
the size arithmetic or the error-message formatting; the driver fails if a
call is not refused on the host.  Skipped where a GPU is visible (the
driver's pointers are host memory) or hipcc / g++ are absent.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

from fastkernels_amd import build as fk_build

ROOT = Path(__file__).resolve().parents[1]
DRIVER = ROOT / "tests" / "asan" / "fk_abi_asan.cpp"

# host-side instrumentation only: -Xarch_host directly before each -fsanitize
ASAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]


def _compile(src: Path, obj: Path) -> subprocess.CompletedProcess:
    flags = [f for f in fk_build.HIPCC_FLAGS if f != "-O3"] + ["-O1", "-g"]
    cmd = [fk_build._hipcc(), *flags, *ASAN_HOST, f"-I{fk_build.INCLUDE}", f"-I{fk_build.CSRC}", "-c", str(src), "-o", str(obj)]
    return subprocess.run(cmd, capture_output=True, text=True)


@pytest.mark.skipif(torch.cuda.is_available(), reason="host-only check: its pointers are host memory")
@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not found")
def test_c_abi_host_validation_under_asan(tmp_path):
    try:
        fk_build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not found")
    srcs = [*fk_build.sources(), DRIVER]
    objs = [tmp_path / (s.stem + ".o") for s in srcs]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        results = list(ex.map(_compile, srcs, objs))
    for s, r in zip(srcs, results):
        assert r.returncode == 0, f"{s.name}: {r.stderr[-2000:]}"
    exe = tmp_path / "fk_abi_asan"
    rocm_lib = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "lib"
    link = ["g++", "-fsanitize=address", *map(str, objs), f"-L{rocm_lib}", "-lamdhip64", f"-Wl,-rpath,{rocm_lib}", "-o", str(exe)]
    r = subprocess.run(link, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    assert " 0 not refused" in r.stdout, r.stdout
