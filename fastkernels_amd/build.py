"""Build libfastkernels_hip.so (the gfx950 HIP kernels + C ABI) in-tree.

Usage: ``python -m fastkernels_amd.build`` (or ``fastkernels_amd.build.build()``);
``--timeline`` builds the diagnostic phase-timeline variant alongside.
Each ``csrc/*.hip`` file is compiled to an object with hipcc for
``--offload-arch=gfx950`` and the objects are linked into
``fastkernels_amd/libfastkernels_hip.so``.  Compilation runs on a machine
without a GPU (hipcc cross-compiles).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
LIB_NAME = "libfastkernels_hip.so"
LIB_PATH = PACKAGE_DIR / LIB_NAME
TIMELINE_LIB_PATH = PACKAGE_DIR / "libfastkernels_hip_timeline.so"
BUILD_DIR = PACKAGE_DIR / "_build"
ARCH = "gfx950"

# Packed-fp32 VALU ops are disabled for all device code: hipcc still
# vectorises fp32 math, but without the v_pk_*_f32 forms.
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-mcode-object-version=5",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; the HIP kernels cannot be built")
    return found


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the disabled device
    # feature; that line is expected noise.
    noise = "packed-fp32-ops"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False, jobs: int | None = None, timeline: bool = False) -> Path:
    """Compile every kernel source and link the shared library; returns its path.

    ``timeline=True`` builds the diagnostic variant instead: the single-launch
    kernels record per-phase wall-clock markers (``-DFK_TIMELINE``) into
    ``libfastkernels_hip_timeline.so``, read by ``python -m
    fastkernels_amd.timeline``.  The product library is left untouched."""

    hipcc = _hipcc()
    build_dir = BUILD_DIR / "timeline" if timeline else BUILD_DIR
    out_path = TIMELINE_LIB_PATH if timeline else LIB_PATH
    build_dir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    extra = ["-DFK_TIMELINE"] if timeline else []

    def compile_one(src: Path) -> Path:
        obj = build_dir / (src.stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, *extra, f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd))
        _run(cmd)
        return obj

    workers = jobs or min(len(srcs), os.cpu_count() or 1, 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(compile_one, srcs))

    tmp = out_path.with_name(out_path.name + ".tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(tmp, out_path)
    return out_path


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv, timeline="--timeline" in sys.argv)
    print(path)
