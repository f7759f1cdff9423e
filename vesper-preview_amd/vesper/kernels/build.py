"""Build ``libvesper_kernels.so`` from ``csrc/`` with hipcc for gfx950, in-tree.

Usage: ``python -m vesper.kernels.build`` (from ``vesper-preview_amd/``) or ``build()`` from Python.
Each source compiles to its own object under ``_build/`` in parallel, then one shared library is
linked next to this file, where ``vesper.kernels._lib`` loads it. No torch extension machinery is
involved: the library's interface is the C ABI declared in ``include/vesper_kernels.h``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parents[2] / "include"
OBJDIR = HERE / "_build"
LIBRARY = HERE / "libvesper_kernels.so"
# bench.py's HBM streaming probes: measurement only, kept out of the mixers' library
PROBE_SOURCE = HERE / "probe" / "hbm_probe.hip"
PROBE_LIBRARY = HERE / "libvesper_probe.so"
ARCH = os.environ.get("VSP_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops off: hipcc must not emit packed fp32 VALU forms in these kernels
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: the kernels need ROCm's hipcc to build")
    return found


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path) -> Path:
    obj = OBJDIR / (src.stem + src.suffix.replace(".", "_") + ".o")
    cmd = [hipcc(), *HIP_FLAGS, "-I", str(CSRC), "-I", str(INCLUDE), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True, check=False)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr[-6000:]}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every source in ``csrc/`` and link ``libvesper_kernels.so``; returns its path."""
    OBJDIR.mkdir(exist_ok=True)
    srcs = sources()
    workers = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    # --no-undefined: a kernel whose host stub failed to instantiate must fail the build, not the load
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True, check=False)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-6000:]}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(srcs)} sources", file=sys.stderr)
    build_probe()
    return LIBRARY


def build_probe() -> Path:
    """Compile bench.py's HBM streaming probes into ``libvesper_probe.so``; returns its path."""
    tmp = PROBE_LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIP_FLAGS, "-shared", "-Wl,--no-undefined", "-o", str(tmp), str(PROBE_SOURCE)]
    proc = subprocess.run(cmd, capture_output=True, text=True, check=False)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {PROBE_SOURCE.name}:\n{proc.stderr[-6000:]}")
    os.replace(tmp, PROBE_LIBRARY)
    return PROBE_LIBRARY


if __name__ == "__main__":
    build(verbose=True)
