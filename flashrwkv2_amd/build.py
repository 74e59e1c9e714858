"""Builds the gfx950 WKV7 library in-tree: flashrwkv2_amd/lib/libflashrwkv2_amd.so.

Every ``csrc/*.hip`` file is compiled by ``hipcc --offload-arch=gfx950`` into
an object, then linked into one shared library with a plain C ABI
(``include/flashrwkv2_amd.h``).  Run ``python -m flashrwkv2_amd.build``.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "lib"
LIB_NAME = "libflashrwkv2_amd.so"
OBJ_DIR = PKG / "_build"

ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    # Packed fp32 VALU forms are disabled for every kernel in this library.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build flashrwkv2_amd")
    return path


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


FASTCALL_SRC = CSRC / "fastcall.c"


def fastcall_name() -> str:
    import sysconfig

    return "_fastcall" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so")


def _build_fastcall(lib: Path) -> Path:
    """The CPython fast-call module over the library (plain C, linked to the
    library with an $ORIGIN rpath, so both load from flashrwkv2_amd/lib)."""
    import sysconfig

    out = LIB_DIR / fastcall_name()
    tmp = LIB_DIR / (out.name + ".tmp")
    cc = shutil.which("gcc") or "cc"
    cmd = [cc, "-O2", "-shared", "-fPIC", "-Wall", f"-I{sysconfig.get_paths()['include']}",
           str(FASTCALL_SRC), f"-L{LIB_DIR}", f"-l:{lib.name}", "-Wl,-rpath,$ORIGIN",
           "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"fastcall build failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    return out


HOSTPATH_SRC = CSRC / "hostpath.cpp"


def hostpath_name() -> str:
    import sysconfig

    return "_hostpath" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so")


def _hostpath_flags() -> list[str]:
    import sysconfig

    import torch
    import torch.utils.cpp_extension as cpp

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return ["-O2", "-fPIC", "-std=c++17", "-Wall", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
            "-DTORCH_EXTENSION_NAME=_hostpath", "-D__HIP_PLATFORM_AMD__",
            *(f"-I{d}" for d in cpp.include_paths()), f"-I{sysconfig.get_paths()['include']}",
            "-I/opt/rocm/include"]


def _compile_hostpath() -> Path:
    """The torch C++ extension of the per-step fast path (g++ against torch's
    headers; no HIP code in it: it calls the library's C ABI)."""
    obj = OBJ_DIR / "hostpath.o"
    cxx = shutil.which("g++") or "c++"
    cmd = [cxx, *_hostpath_flags(), "-c", str(HOSTPATH_SRC), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hostpath compile failed:\n{proc.stdout}\n{proc.stderr}")
    return obj


def _link_hostpath(obj: Path, lib: Path) -> Path:
    import torch.utils.cpp_extension as cpp

    out = LIB_DIR / hostpath_name()
    tmp = LIB_DIR / (out.name + ".tmp")
    cxx = shutil.which("g++") or "c++"
    cmd = [cxx, "-shared", "-fPIC", str(obj), *(f"-L{d}" for d in cpp.library_paths()),
           "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", f"-L{LIB_DIR}", f"-l:{lib.name}",
           "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hostpath link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = True) -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    workers = min(len(sources), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(workers + 1) as pool:
        host_obj = pool.submit(_compile_hostpath)   # the longest compile: start it first
        objects = list(pool.map(_compile, sources))
        host_obj = host_obj.result()
    out = LIB_DIR / LIB_NAME
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,-soname,{LIB_NAME}",
           "-o", str(tmp),
           *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    fast = _build_fastcall(out)
    host = _link_hostpath(host_obj, out)
    if verbose:
        print(f"built {out}, {fast.name} and {host.name}", file=sys.stderr)
    return out


if __name__ == "__main__":
    build()
