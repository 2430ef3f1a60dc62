"""Builds ``libomniasr_mi355x.so`` (the gfx950 kernels behind the C ABI of include/omniasr_mi355x.h).

Every ``.hip`` file of this directory is compiled by ``hipcc`` for gfx950 only and linked into one
shared library next to the package; ``python build.py`` or :func:`build` (called by
``__graft_entry__.build``).  No GPU is needed: hipcc cross-compiles.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PACKAGE = HERE.parent
ROOT = PACKAGE.parent
LIBRARY = PACKAGE / "libomniasr_mi355x.so"
ARCH = "gfx950"

# Packed-fp32 instructions (v_pk_*_f32) stay off: ordinary float code is compiled without them.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
         f"-I{ROOT / 'include'}"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the HIP kernels cannot be built")
    return path


def sources() -> list[Path]:
    return sorted(HERE.glob("*.hip"))


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *FLAGS, *DEVICE_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile every kernel source and link the library (always rebuilds)."""
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    objs = [objdir / (s.stem + ".o") for s in sources()]
    jobs = max(1, min(len(objs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(lambda so: _compile(*so), zip(sources(), objs)))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking {LIBRARY.name} failed:\n{res.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(objs)} sources", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
