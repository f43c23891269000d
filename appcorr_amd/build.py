"""Build liboudjat_hip.so, the gfx950 C-ABI library, in-tree.

Every `csrc/*.hip` is compiled to an object under `_build/` (in parallel) and linked into
`appcorr_amd/liboudjat_hip.so`. The library is loaded with ctypes by `appcorr_amd._lib`; there is no
Python extension module and no JIT step.

Run as `python -m appcorr_amd.build` or call `build()`.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "liboudjat_hip.so"
ARCH = "gfx950"

# Packed-fp32 instruction selection is disabled for all device code: the compiler still emits
# scalar or float2 fp32 arithmetic, but no v_pk_* fp32 instructions, whose results have been unreliable
# on this hardware.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm at /opt/rocm)")


def _compile(src: Path, obj: Path) -> tuple[Path, str]:
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    log = "\n".join(
        line
        for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line  # the host pass does not know the device feature
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{log}")
    return obj, log


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 and link the shared library. Always rebuilds."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    objs = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, BUILD_DIR / (s.stem + ".o")) for s in sources]
        for f in futs:
            obj, log = f.result()
            objs.append(obj)
            if verbose and log.strip():
                print(log, file=sys.stderr)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
