"""Build the native parts of xtile_amd in-tree.

Produces, under ``xtile_amd/lib/``:
  * ``libxtile_amd.so`` - the C ABI of ``include/xtile_amd.h``: xt parser,
    verifier, passes, launch planner and the gfx950 HIP kernels;
  * ``xt-opt``          - the command-line driver (host code only);
  * ``_xtile<ext>.so``   - the compiled Python module ``_xtile``
    (``csrc/XTModule.cpp``, pybind11) over the C ABI, with the reference
    module's function names;
  * ``libxt_ceiling.so`` - the measurement kernels of ``include/xt_ceiling.h``
    (a copy, an empty kernel and an MFMA loop) that bench.py times for its
    ceilings; the tile programs never use it.

Usage: ``python xtile_amd/build.py`` (or ``__graft_entry__.build()``); it runs
without importing the package, whose __init__ needs the library it builds.
Every call recompiles everything.
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
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
OBJ = PKG / "lib" / "obj"

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
CXX = shutil.which("g++") or "g++"
ARCH = "gfx950"

HOST_SOURCES = ["ir.cpp", "verify.cpp", "passes.cpp", "plan.cpp", "fused.cpp", "staged.cpp", "to_nova.cpp"]
KERNEL_SOURCES = ["kernels/elementwise.hip", "kernels/gemm.hip", "kernels/conv.hip", "kernels/conv_general.hip", "kernels/conv_igemm.hip", "kernels/conv_image.hip", "kernels/conv_small.hip",
                  "kernels/tilevm.hip", "kernels/fused_jit.cpp"]
HOST_FLAGS = ["-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter"]
# Packed-FP32 instruction forms are disabled for every HIP compile.
HIP_FLAGS = [
    "-std=c++17",
    "-O3",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; drop that notice
    lines = [
        line
        for line in proc.stdout.splitlines()
        if "is not a recognized feature for this target" not in line
    ]
    if proc.returncode != 0:
        raise RuntimeError("build step failed: " + " ".join(cmd) + "\n" + "\n".join(lines))
    if lines:
        print("\n".join(lines), file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile libxtile_amd.so and xt-opt; returns the library path."""
    OBJ.mkdir(parents=True, exist_ok=True)
    jobs = []
    host_objs = []
    for src in HOST_SOURCES:
        obj = OBJ / (Path(src).stem + ".o")
        host_objs.append(obj)
        jobs.append([CXX, *HOST_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    rt_obj = OBJ / "runtime.o"
    jobs.append(
        [HIPCC, *HIP_FLAGS, "-c", str(CSRC / "runtime.cpp"), "-o", str(rt_obj)]
    )
    kern_objs = []
    for src in KERNEL_SOURCES:
        obj = OBJ / (Path(src).stem + ".o")
        kern_objs.append(obj)
        jobs.append([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    ceil_obj = OBJ / "ceiling.o"
    jobs.append([HIPCC, *HIP_FLAGS, "-c", str(CSRC / "ceiling.hip"), "-o", str(ceil_obj)])
    xt_opt_obj = OBJ / "xt_opt.o"
    jobs.append([CXX, *HOST_FLAGS, "-c", str(CSRC / "xt_opt.cpp"), "-o", str(xt_opt_obj)])

    workers = min(8, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for cmd in jobs:
            if verbose:
                print(" ".join(cmd))
        list(pool.map(_run, jobs))

    lib = LIB / "libxtile_amd.so"
    tmp = LIB / "libxtile_amd.so.tmp"
    _run(
        [
            HIPCC,
            "-shared",
            "-fPIC",
            f"--offload-arch={ARCH}",
            *map(str, host_objs),
            str(rt_obj),
            *map(str, kern_objs),
            f"-L{ROCM}/lib",
            "-lhiprtc",
            f"-Wl,-rpath,{ROCM}/lib",
            "-o",
            str(tmp),
        ]
    )
    os.replace(tmp, lib)
    ceil_tmp = LIB / "libxt_ceiling.so.tmp"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", str(ceil_obj), "-o", str(ceil_tmp)])
    os.replace(ceil_tmp, LIB / "libxt_ceiling.so")
    _run([CXX, *map(str, host_objs), str(xt_opt_obj), "-o", str(LIB / "xt-opt")])
    build_module()
    return lib


def module_path() -> Path:
    """Where build_module() puts the compiled ``_xtile`` module."""
    return LIB / ("_xtile" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))


def build_module() -> Path:
    """Compile csrc/XTModule.cpp against the freshly linked libxtile_amd.so
    (found beside it at run time through an $ORIGIN rpath)."""
    import pybind11

    out = module_path()
    tmp = out.with_name(out.name + ".tmp")
    _run(
        [
            CXX,
            *HOST_FLAGS,
            "-shared",
            "-fvisibility=hidden",
            f"-I{pybind11.get_include()}",
            f"-I{sysconfig.get_paths()['include']}",
            f"-I{ROOT / 'include'}",
            str(CSRC / "XTModule.cpp"),
            f"-L{LIB}",
            "-lxtile_amd",
            "-Wl,-rpath,$ORIGIN",
            "-o",
            str(tmp),
        ]
    )
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
