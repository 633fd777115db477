"""Build the reference's own C++ scheduler/allocator/prefix cache as a checker.

Test infrastructure only. Compiles, from the sources where they lie under
/root/reference/engine (block_allocator.cpp, sequence.cpp, scheduler.cpp,
prefix_cache.cpp and the pybind11 module bindings.cpp -- standard C++17 and
pybind11 headers, nothing generated), one extension module into
``oracle/_ref/memforge_c.<abi>.so``. Tests load it under the name
``memforge_c`` from that path and drive it side by side with
``memforge_amd.memforge_c`` on the same scripted workloads.

Nothing is copied: g++ reads the reference files in place and writes only
under oracle/_ref/ (git-ignored). Without /root/reference (the GPU box) this
is a no-op and the differential tests skip.
"""

from __future__ import annotations

import subprocess
import sys
import sysconfig
from pathlib import Path

REF_ENGINE = Path("/root/reference/engine")
OUT_DIR = Path(__file__).resolve().parent / "_ref"
SOURCES = ["block_allocator.cpp", "sequence.cpp", "scheduler.cpp", "prefix_cache.cpp", "bindings.cpp"]


def module_path() -> Path:
    return OUT_DIR / ("memforge_c" + sysconfig.get_config_var("EXT_SUFFIX"))


def build(verbose: bool = False) -> Path | None:
    if not (REF_ENGINE / "src").is_dir():
        return None
    import pybind11

    OUT_DIR.mkdir(parents=True, exist_ok=True)
    out = module_path()
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
           f"-I{REF_ENGINE / 'include'}", f"-I{pybind11.get_include()}",
           f"-I{sysconfig.get_paths()['include']}",
           *[str(REF_ENGINE / "src" / s) for s in SOURCES], "-o", str(out)]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    return out


def load():
    """The reference module, or None if it is not built."""
    import importlib.util

    path = module_path()
    if not path.exists():
        return None
    spec = importlib.util.spec_from_file_location("memforge_c", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


if __name__ == "__main__":
    p = build(verbose=True)
    print(p if p else "reference engine sources not present; nothing built")
    sys.exit(0)
