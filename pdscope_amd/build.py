"""Build libpdscope_moe.so (gfx950) and the host extension modules in-tree.

    python -m pdscope_amd.build          # or __graft_entry__.build()

Every .hip file under pdscope_amd/csrc is compiled to an object in
pdscope_amd/_build/ (in parallel), then linked into
pdscope_amd/libpdscope_moe.so next to this file.  The CPython extension
module pdscope_layer_dispatch (csrc/layer_dispatch_module.cpp, host code only)
is compiled with the host C++ compiler into
pdscope_amd/pdscope_layer_dispatch<EXT_SUFFIX>; it loads the HIP library at
import.  pdscope_amd._records (csrc/records_module.cpp, host code only) is the
C base type of the ledger's key records.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libpdscope_moe.so"
ARCH = os.environ.get("PDSCOPE_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-munsafe-fp-atomics",
    # never emit packed fp32 ops (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{CSRC}",
    f"-I{PKG.parent / 'include'}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the gfx950 library cannot be built")
    return path


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr[-6000:]}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    for mod in (build_dispatch_module(), build_records_module()):
        if verbose:
            print(f"built {mod}", file=sys.stderr)
    return LIB


_EXT = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
DISPATCH_SRC = CSRC / "layer_dispatch_module.cpp"
DISPATCH_MODULE = PKG / ("pdscope_layer_dispatch" + _EXT)
RECORDS_SRC = CSRC / "records_module.cpp"
RECORDS_MODULE = PKG / ("_records" + _EXT)


def _build_host_module(src: Path, out: Path, libs=()) -> Path:
    """One CPython extension module from one C++ source (host code only)."""
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError(f"no host C++ compiler for the {out.name} extension")
    tmp = out.with_name(out.name + ".tmp")
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wextra",
           f"-I{sysconfig.get_paths()['include']}", str(src), "-o", str(tmp), *libs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"{out.name} build failed:\n{proc.stderr[-6000:]}")
    os.replace(tmp, out)
    return out


def build_dispatch_module() -> Path:
    """The pdscope_layer_dispatch extension (plain CPython API, no GPU code)."""
    return _build_host_module(DISPATCH_SRC, DISPATCH_MODULE, ["-ldl"])


def build_records_module() -> Path:
    """pdscope_amd._records, the ledger's record base type (plain CPython API)."""
    return _build_host_module(RECORDS_SRC, RECORDS_MODULE)


if __name__ == "__main__":
    build(verbose=True)
