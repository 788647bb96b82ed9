"""Build the gfx950 C-ABI library and its pybind11 binding, in tree.

    python -m sili__new_amd.build          # or __graft_entry__.build()

Outputs (git-ignored, shipped with the tree to the GPU box):
    sili__new_amd/libsili_hip.so              HIP kernels + C ABI (include/sili_hip.h)
    sili__new_amd/_sili_hip<ext-suffix>.so    pybind11 module over the C ABI
Intermediate objects go to sili__new_amd/_build/.

Every HIP translation unit is compiled with packed-FP32 instructions disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shlex
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "_build"
LIB = PKG / "libsili_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("SILI_OFFLOAD_ARCH", "gfx950")

HIP_SOURCES = ["kernels.hip", "stream.hip", "build.hip", "synapto.hip", "policy.hip", "gen.hip", "train.hip",
               "csr_util.hip", "for_index.hip", "tile_enc.hip", "layout.hip", "b4res.hip", "push.hip", "patch.hip", "staged.hip", "capi.hip"]

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-parameter",
    f"-I{CSRC}", f"-I{REPO / 'include'}",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(shlex.quote(c) for c in cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed ({r.returncode}): {cmd[0]} ... {cmd[-1]}")
    # the host pass does not know the gfx target feature; that warning is noise
    noise = ("packed-fp32-ops", "warning generated", "warnings generated")
    text = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if l.strip() and not any(n in l for n in noise))
    if text and verbose:
        sys.stderr.write(text + "\n")


def _compile(src: str, verbose: bool) -> Path:
    obj = OUT / (Path(src).stem + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)], verbose)
    return obj


def build_library(verbose: bool = False, jobs: int | None = None) -> Path:
    OUT.mkdir(exist_ok=True)
    jobs = jobs or min(len(HIP_SOURCES), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), HIP_SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_binding(verbose: bool = False) -> Path:
    import pybind11

    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = PKG / f"_sili_hip{suffix}"
    tmp = out.with_name(out.name + ".tmp")
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-shared", "-fPIC",
        f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}",
        f"-I{REPO / 'include'}",
        str(CSRC / "pymod.cpp"), "-o", str(tmp),
        f"-L{PKG}", "-lsili_hip", "-Wl,-rpath,$ORIGIN",
    ]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> None:
    build_library(verbose)
    build_binding(verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", LIB)
