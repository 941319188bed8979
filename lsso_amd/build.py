"""Build the gfx950 native library in-tree with hipcc.

Usage: ``python -m lsso_amd.build`` (or ``lsso_amd.build.build_library()``).
The shared library lands in ``lsso_amd/_lib/liblsso_hip_gfx950.so``; object
files go to ``_build/`` at the repository root.  Each translation unit is
compiled in its own hipcc process, then linked once.  The benchmark's HBM
probes (``lsso_probe.hip``, not part of the mixer's C ABI) are linked into
their own ``liblsso_probe_gfx950.so`` beside it.
"""

from __future__ import annotations

import concurrent.futures
import os
from pathlib import Path
import shutil
import subprocess

PACKAGE_ROOT = Path(__file__).resolve().parent
REPOSITORY_ROOT = PACKAGE_ROOT.parent
SOURCE_DIR = PACKAGE_ROOT / "csrc"
INCLUDE_DIR = REPOSITORY_ROOT / "include"
OUTPUT_DIR = PACKAGE_ROOT / "_lib"
OBJECT_DIR = REPOSITORY_ROOT / "_build"
OFFLOAD_ARCH = "gfx950"
LIBRARY_NAME = f"liblsso_hip_{OFFLOAD_ARCH}.so"
SOURCES = (
    "lsso_capi.hip",
    "lsso_mixer.hip",
    "lsso_linear.hip",
    "lsso_linear_grad.hip",
    "lsso_fused.hip",
    "lsso_backward.hip",
    "lsso_project_reduce.hip",
    "lsso_weight_grad.hip",
)
PROBE_SOURCE = "lsso_probe.hip"
PROBE_LIBRARY_NAME = f"liblsso_probe_{OFFLOAD_ARCH}.so"

# Packed FP32 VALU forms (v_pk_add/mul/fma_f32) are disabled for all device
# code: some of their forms have returned wrong results on the MI355X boxes
# this library is tested on, without any error.  hipcc's host pass warns that
# it does not know the feature, which is harmless.
DEVICE_FLAGS = (
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


def library_path() -> Path:
    return OUTPUT_DIR / LIBRARY_NAME


def probe_library_path() -> Path:
    return OUTPUT_DIR / PROBE_LIBRARY_NAME


def _hipcc() -> str:
    candidate = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(candidate).exists():
        raise RuntimeError("hipcc was not found; the gfx950 library cannot be built")
    return candidate


def _run(command: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(command), flush=True)
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(
            "hipcc failed (" + " ".join(command) + "):\n" + result.stdout + result.stderr
        )


def build_library(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source for gfx950 and link the shared library."""

    hipcc = _hipcc()
    OBJECT_DIR.mkdir(parents=True, exist_ok=True)
    OUTPUT_DIR.mkdir(parents=True, exist_ok=True)
    include = [f"-I{INCLUDE_DIR}", f"-I{SOURCE_DIR}"]
    commands = []
    objects = []
    for source in SOURCES:
        obj = OBJECT_DIR / (source + ".o")
        objects.append(obj)
        commands.append(
            [hipcc, *DEVICE_FLAGS, *include, "-c", str(SOURCE_DIR / source), "-o", str(obj)]
        )
    probe_object = OBJECT_DIR / (PROBE_SOURCE + ".o")
    commands.append(
        [hipcc, *DEVICE_FLAGS, "-c", str(SOURCE_DIR / PROBE_SOURCE), "-o", str(probe_object)]
    )
    workers = jobs or min(len(commands), os.cpu_count() or 1, 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        for future in [pool.submit(_run, command, verbose) for command in commands]:
            future.result()
    for linked, output in ((objects, library_path()), ([probe_object], probe_library_path())):
        temporary = output.with_suffix(".so.tmp")
        _run(
            [hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC",
             *[str(o) for o in linked], "-o", str(temporary)],
            verbose,
        )
        os.replace(temporary, output)
    return library_path()


if __name__ == "__main__":
    print(build_library(verbose=True))
