"""Build libnanoengine_hip.so for gfx950 with hipcc (in-tree, no JIT cache).

``python inference-engine-from-scratch_amd/build.py`` compiles every ``csrc/*.hip``
into ``nanoengine_amd/libnanoengine_hip.so``.  hipcc cross-compiles, so this runs
on a machine without a GPU.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
OUTPUT = PACKAGE_DIR / "nanoengine_amd" / "libnanoengine_hip.so"
BUILD_DIR = PACKAGE_DIR / "_build"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # packed fp32 VALU forms stay off: plain float code must not become v_pk_*_f32
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build")
    return found


def compile_one(source: Path) -> Path:
    obj = BUILD_DIR / (source.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{result.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        objects = list(pool.map(compile_one, sources))
    tmp = OUTPUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp)]
    cmd += [str(o) for o in objects]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, OUTPUT)
    if verbose:
        print(f"built {OUTPUT}")
    build_host_step(verbose)
    return OUTPUT


def build_host_step(verbose: bool = False) -> Path:
    """The CPython extension of the verify step's host bookkeeping (csrc/host_step.c)."""
    import sysconfig

    out = PACKAGE_DIR / "nanoengine_amd" / ("_host_step" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_name(out.name + ".tmp")
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("gcc not found; it builds the host-step extension")
    cmd = [cc, "-O2", "-shared", "-fPIC", "-std=c11", "-Wall", f"-I{sysconfig.get_paths()['include']}",
           str(CSRC / "host_step.c"), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"gcc failed on host_step.c:\n{result.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
