"""Build libinfengine_amd.so for gfx950 with hipcc, in-tree.

Every csrc/*.hip and csrc/*.cpp file is compiled to an object under
infengine_amd/_build/ (in parallel) and linked into
infengine_amd/libinfengine_amd.so, which the package loads with ctypes.

    python infengine_amd/build.py

(run it as a script: importing the package loads the library it is rebuilding)
"""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent
SRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libinfengine_amd.so"
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
    # packed fp32 (v_pk_*_f32) is kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{SRC}",
]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: drop that noise
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build(jobs: int | None = None) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(SRC.glob("*.hip")) + sorted(SRC.glob("*.cpp"))
    if not sources:
        raise RuntimeError(f"no sources under {SRC}")

    def compile_one(src: pathlib.Path) -> pathlib.Path:
        obj = BUILD / (src.stem + ".o")
        lang = ["-x", "hip"] if src.suffix == ".hip" else []
        _run([HIPCC, *FLAGS, *lang, "-c", str(src), "-o", str(obj)])
        return obj

    jobs = jobs or min(8, os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, sources))
    tmp = LIB.with_suffix(".so.tmp")
    # -z defs: an unresolved symbol (e.g. a kernel whose host stub was not emitted) fails
    # the build instead of the first dlopen
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", *map(str, objs),
          "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
