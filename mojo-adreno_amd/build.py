"""Build libaq.so (HIP kernels for gfx950 + the C ABI) in-tree, next to the Python package.

    python mojo-adreno_amd/build.py            # compiles every source, links aq/libaq.so
    python mojo-adreno_amd/build.py --changed  # only sources newer than their object (or than a header)

Each source is compiled with hipcc for --offload-arch=gfx950 (no other target); objects go to _build/ beside this
file. Packed-FP32 instructions are disabled for device code (-Xclang -target-feature -Xclang -packed-fp32-ops).
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
OUT = HERE / "aq" / "libaq.so"
BUILD = HERE / "_build"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libaq.so)")


COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function", "-Wno-unused-result"]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


# Per-source device flags. The MFMA kernels keep their accumulators in ordinary VGPRs: with AGPR accumulators the
# register allocator rotates them through copies every loop iteration.
EXTRA = {"aq_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    if src.suffix == ".hip":
        cmd = [hipcc(), *DEVICE, *EXTRA.get(src.name, []), *COMMON, "-c", str(src), "-o", str(obj)]
    else:  # host-only C++ (format converters, status text): the system compiler, no device pass
        cmd = ["g++", *COMMON, "-ffp-contract=off", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}{r.stderr}")
    return obj


def _stale(src: Path, headers: list) -> bool:
    obj = BUILD / (src.name + ".o")
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    return src.stat().st_mtime > t or any(h.stat().st_mtime > t for h in headers)


def build(verbose: bool = False, changed_only: bool = False) -> Path:
    """Compile every source (changed_only: only those newer than their object or than any header) and link."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    headers = sorted(CSRC.glob("*.h")) + sorted((HERE.parent / "include").glob("*.h"))
    todo = [s for s in sources if _stale(s, headers)] if changed_only else sources
    with ThreadPoolExecutor(max_workers=max(1, min(8, len(todo)))) as ex:
        list(ex.map(_compile, todo))
    objs = [BUILD / (s.name + ".o") for s in sources]
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(sources)} sources ({len(todo)} compiled)")
    return OUT


if __name__ == "__main__":
    build(verbose=True, changed_only="--changed" in sys.argv[1:])
    sys.exit(0)
