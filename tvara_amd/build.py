"""Build libtvara_capi.so for gfx950 with hipcc, in-tree.

The library goes to build/release/libtvara_capi.so, the path the reference's
ctypes loader searches (python/tvara/native.py:17-23).  Every source compiles
for gfx950 only, with packed-FP32 instruction selection disabled.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "tvara_amd" / "csrc"
INCLUDE = ROOT / "include"
OUT_DIR = ROOT / "build" / "release"
LIBRARY = OUT_DIR / "libtvara_capi.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def sources():
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path, obj: Path, verbose: bool):
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [HIPCC, *FLAGS, *lang, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr[-8000:]}")
    return res.stderr


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source for gfx950 and link the shared library."""
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    objs = [obj_dir / (s.name + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(jobs) as pool:
        futures = [pool.submit(_compile, s, o, verbose) for s, o in zip(srcs, objs)]
        for f in futures:
            warnings = f.result()
            if verbose and warnings.strip():
                print(warnings, file=sys.stderr)
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-8000:]}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
