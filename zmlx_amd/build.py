"""Build ``libzmlx_amd.so`` (gfx950) from ``zmlx_amd/csrc/*.hip`` with hipcc.

Usage: ``python -m zmlx_amd.build`` (or ``zmlx_amd.build.build()``).  The
library is written in-tree to ``zmlx_amd/_lib/`` so that it travels with the
source tree; nothing is installed elsewhere.
"""

from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
OUT_DIR = PKG / "_lib"
LIB_NAME = "libzmlx_amd.so"
ARCH = os.environ.get("ZMOE_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=fast-honor-pragmas",
    # packed fp32 VALU ops are disabled for all device code of this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def source_hash() -> str:
    """Hash of the library's sources (csrc/*.hip, csrc/*.h and the public
    header), compiled into zmoe_version() so a loaded library can be checked
    against the tree it is loaded from."""
    h = hashlib.sha256()
    files = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")) + [INCLUDE / "zmlx_amd.h"]
    for f in files:
        h.update(f.name.encode())
        h.update(b"\0")
        h.update(f.read_bytes())
        h.update(b"\0")
    return h.hexdigest()[:16]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _compile(src: Path, obj: Path, extra: list[str]) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    extra = list(extra_flags or []) + [f'-DZMOE_SOURCE_HASH="{source_hash()}"']
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [obj_dir / (s.stem + ".o") for s in srcs]
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_compile, s, o, extra) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    lib = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


if __name__ == "__main__":
    build(verbose=True, extra_flags=sys.argv[1:])
