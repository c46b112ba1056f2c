"""Build libtvara_capi.so for gfx950, in-tree.

The library goes to build/release/libtvara_capi.so, the path the reference's
ctypes loader searches (python/tvara/native.py:17-23).  The build is the
repository's CMakeLists.txt (HIP language, ROCm clang, gfx950 only, packed-FP32
instruction selection disabled), configured into build/release with Ninja.
Where cmake is absent the same flags drive hipcc directly.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
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
    "-Wextra",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def sources():
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _run(cmd, verbose):
    if verbose:
        print(" ".join(map(str, cmd)), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        out = res.stdout + res.stderr
        errors = "\n".join(line for line in out.splitlines() if "error" in line or "FAILED" in line)
        raise RuntimeError(f"{cmd[0]} failed:\n{errors[-8000:]}\n--- tail ---\n{out[-3000:]}")
    return res


def build_cmake(verbose: bool = False, jobs: int | None = None) -> Path:
    """Configure (once) and build every source with CMake; always recompiles."""
    jobs = jobs or min(os.cpu_count() or 4, 8)
    generator = ["-G", "Ninja"] if shutil.which("ninja") else []
    cache = OUT_DIR / "CMakeCache.txt"
    if cache.exists() and "Ninja" not in cache.read_text(errors="ignore") and generator:
        shutil.rmtree(OUT_DIR)  # a tree configured by another generator
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    _run(["cmake", "-S", str(ROOT), "-B", str(OUT_DIR), *generator, "-DCMAKE_BUILD_TYPE=Release"], verbose)
    # a failed build raises and leaves the previous library in place
    keep = LIBRARY.with_suffix(".so.prev")
    if LIBRARY.exists():
        os.replace(LIBRARY, keep)
    try:
        _run(["cmake", "--build", str(OUT_DIR), "--clean-first", "-j", str(jobs)], verbose)
    except RuntimeError:
        if keep.exists() and not LIBRARY.exists():
            os.replace(keep, LIBRARY)
        raise
    if not LIBRARY.exists():
        raise RuntimeError(f"cmake built no {LIBRARY}")
    keep.unlink(missing_ok=True)
    return LIBRARY


# per-source flags, as CMakeLists.txt sets them
SOURCE_FLAGS = {"model_kernels.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: Path, obj: Path, verbose: bool):
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    extra = SOURCE_FLAGS.get(src.name, [])
    return _run([HIPCC, *FLAGS, *extra, *lang, "-c", str(src), "-o", str(obj)], verbose).stderr


def build_hipcc(verbose: bool = False, jobs: int | None = None) -> Path:
    """The same build with hipcc alone (hosts without cmake)."""
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
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, LIBRARY)
    return LIBRARY


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source for gfx950 and link the shared library."""
    if shutil.which("cmake"):
        return build_cmake(verbose, jobs)
    return build_hipcc(verbose, jobs)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
