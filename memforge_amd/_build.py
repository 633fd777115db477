"""Builds the package's native libraries in-tree.

* ``libmemforge_hip.so`` -- the gfx950 device library behind the C ABI in
  ``include/memforge_hip.h``, compiled with ``hipcc --offload-arch=gfx950``.
* ``memforge_c`` -- the host engine (block allocator, scheduler, prefix cache)
  as a CPython extension built with g++ and pybind11.

Both are written next to this file so they travel with the source tree.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sysconfig
from pathlib import Path
from typing import List

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
HIP_LIB = PKG_DIR / "libmemforge_hip.so"
ENGINE_EXT = PKG_DIR / ("memforge_c" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))

HIP_ARCH = "gfx950"
# Packed FP32 instructions are kept out of every kernel: hipcc would otherwise
# form v_pk_* from ordinary float code.
HIPCC_FLAGS = [
    f"--offload-arch={HIP_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # a kernel's leading scalar / pointer arguments (up to two) arrive in
    # scalar registers instead of being loaded from the argument block: the
    # attention and merge kernels take their work lists first so the first
    # load of a wave does not wait on that block (LLVM's AMDGPU kernel
    # argument preloading; the code object keeps a load path for firmware
    # that does not preload)
    "-mllvm", "-amdgpu-kernarg-preload-count=2",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def _run(cmd: List[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}")


def hip_sources() -> List[Path]:
    return sorted(CSRC.glob("*.hip"))


def build_hip(jobs: int = 8) -> Path:
    """Compile every ``csrc/*.hip`` for gfx950 and link ``libmemforge_hip.so``."""
    hipcc = _hipcc()
    objdir = PKG_DIR / "_build"
    objdir.mkdir(exist_ok=True)
    srcs = hip_sources()
    objs = [objdir / (src.stem + ".o") for src in srcs]

    def compile_one(pair):
        src, obj = pair
        _run([hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)])

    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as pool:
        list(pool.map(compile_one, zip(srcs, objs)))
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={HIP_ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_engine() -> Path:
    """Compile the host engine (``csrc/engine``) into the ``memforge_c`` extension."""
    import pybind11

    engine = CSRC / "engine"
    srcs = sorted(engine.glob("*.cpp"))
    py_inc = sysconfig.get_paths()["include"]
    tmp = ENGINE_EXT.with_suffix(".tmp")
    _run([
        "g++", "-O3", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
        "-fvisibility=hidden",
        f"-I{engine}", f"-I{pybind11.get_include()}", f"-I{py_inc}",
        *map(str, srcs), "-o", str(tmp),
    ])
    os.replace(tmp, ENGINE_EXT)
    return ENGINE_EXT


def build_all(jobs: int = 8) -> None:
    build_hip(jobs)
    if (CSRC / "engine").is_dir():
        build_engine()


if __name__ == "__main__":
    build_all()
    print(f"built {HIP_LIB}")
