"""Builds the native parts of tabby_amd in-tree.

* ``tabby_amd/lib/libtabby_sampler.so`` -- the HIP kernels and the C ABI of
  ``include/tabby_sampler.h``, compiled for gfx950 with hipcc (every ``csrc/*.hip``, one
  object each under ``tabby_amd/_build/``, then linked).
* ``tabby_amd/lib/libtabby_sampler_timeline.so`` -- the same, with the row kernel's phase
  timestamps compiled in (``-DTABBY_TIMELINE``), read by ``bench.py --timeline`` only.
* ``tabby_amd/node/build/tabby_sampler.node`` -- the N-API addon that exposes the C ABI to
  Node (g++ against ``/usr/include/node``), when the Node headers are present.

Run ``python -m tabby_amd.build``. All outputs are rebuilt on every call.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_DIR = os.path.join(PKG, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libtabby_sampler.so")
# The same library with the row kernel's phase timestamps compiled in (TABBY_TIMELINE), for
# `bench.py --timeline`; nothing else loads it.
TIMELINE_LIB_PATH = os.path.join(LIB_DIR, "libtabby_sampler_timeline.so")
OBJ_DIR = os.path.join(PKG, "_build")
NODE_DIR = os.path.join(PKG, "node")
NODE_ADDON = os.path.join(NODE_DIR, "build", "tabby_sampler.node")
NODE_INCLUDE = "/usr/include/node"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = os.environ.get("TABBY_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    # f64 tail: every operation rounds once, in source order (V8 evaluates JS that way).
    "-ffp-contract=off",
    # Packed FP32 instructions are kept out of all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the sampler library cannot be built")


def sources() -> list:
    """Every HIP translation unit of the library (csrc/*.hip), in name order."""
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _link(hipcc: str, objs: list, path: str, verbose: bool) -> None:
    tmp = path + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc (link) failed ({r.returncode}):\n{r.stderr[-6000:]}")
    os.replace(tmp, path)


def build_library(verbose: bool = False) -> str:
    """Compiles each csrc/*.hip to an object in parallel, then links the shared library, and
    the timeline variant (tabby_sampler.hip again with TABBY_TIMELINE, the other objects
    shared)."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    hipcc = _hipcc()
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    jobs = []
    for src in sources():
        obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
        jobs.append(([hipcc, *compile_flags, "-c", "-o", obj, src], obj))
    main_src = os.path.join(CSRC, "tabby_sampler.hip")
    timeline_obj = os.path.join(OBJ_DIR, "tabby_sampler_timeline.o")
    jobs.append(([hipcc, *compile_flags, "-DTABBY_TIMELINE", "-c", "-o", timeline_obj, main_src], timeline_obj))
    procs = []
    for cmd, obj in jobs:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    objs = []
    for cmd, obj, proc in procs:
        _, err = proc.communicate()
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed ({proc.returncode}) on {cmd[-1]}:\n{err[-6000:]}")
        objs.append(obj)
    os.makedirs(LIB_DIR, exist_ok=True)
    main_obj = os.path.join(OBJ_DIR, "tabby_sampler.o")
    _link(hipcc, [o for o in objs if o != timeline_obj], LIB_PATH, verbose)
    _link(hipcc, [o for o in objs if o != main_obj], TIMELINE_LIB_PATH, verbose)
    return LIB_PATH


def build_node_addon(verbose: bool = False) -> str | None:
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        return None
    os.makedirs(os.path.dirname(NODE_ADDON), exist_ok=True)
    tmp = NODE_ADDON + ".tmp"
    cmd = [
        shutil.which("g++") or "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
        "-DNODE_GYP_MODULE_NAME=tabby_sampler", "-D__HIP_PLATFORM_AMD__",
        f"-I{NODE_INCLUDE}", f"-I{INCLUDE}", f"-I{ROCM}/include", "-o", tmp,
        os.path.join(NODE_DIR, "addon.cc"),
        f"-L{LIB_DIR}", "-ltabby_sampler", f"-L{ROCM}/lib", "-lamdhip64",
        "-Wl,-rpath,$ORIGIN/../../lib", f"-Wl,-rpath,{ROCM}/lib",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ (node addon) failed ({r.returncode}):\n{r.stderr[-6000:]}")
    os.replace(tmp, NODE_ADDON)
    return NODE_ADDON


def build(verbose: bool = False) -> None:
    build_library(verbose)
    if os.path.exists(os.path.join(NODE_DIR, "addon.cc")):
        build_node_addon(verbose)


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
    print("built", LIB_PATH)
