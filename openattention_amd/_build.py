"""Build the gfx950 kernel library (``openattention_amd/_lib/liboa_hip.so``) with hipcc.

Every ``csrc/*.hip`` file is compiled to an object with ``hipcc --offload-arch=gfx950`` and the
objects are linked with g++ into one shared library.  The library is linked against the HIP
runtime that ships inside torch (same file name the torch extension libraries resolve), so a
process that imports torch first runs both torch and this library on one HIP runtime.

Flags: -O3, -ffp-contract=off (a fused multiply-add only where the source asks for one:
the decision path is replayed bit for bit by the CPU restatement), packed-fp32 code
generation disabled.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "_lib")
LIBNAME = "liboa_hip.so"
ARCH = os.environ.get("OA_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def lib_path() -> str:
    return os.path.join(LIBDIR, LIBNAME)


def _torch_libdir() -> str:
    import importlib.util
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.origin:
        raise RuntimeError("torch is required to locate the HIP runtime to link against")
    return os.path.join(os.path.dirname(spec.origin), "lib")


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every kernel source and link the shared library; returns its path."""
    os.makedirs(LIBDIR, exist_ok=True)
    objdir = os.path.join(LIBDIR, "obj")
    os.makedirs(objdir, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not srcs:
        raise RuntimeError(f"no kernel sources under {CSRC}")
    hipcc = _hipcc()
    procs = []
    objs = []
    for src in srcs:
        obj = os.path.join(objdir, os.path.basename(src)[:-4] + ".o")
        objs.append(obj)
        cmd = [hipcc, *HIPCC_FLAGS, "-I", CSRC, "-I", INCLUDE, "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        if jobs and len([p for _, p in procs if p.poll() is None]) >= jobs:
            procs[0][1].wait()
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        # the host pass does not know the packed-fp32 target feature; that notice is harmless
        text = "\n".join(ln for ln in text.splitlines() if "packed-fp32-ops" not in ln)
        if p.returncode != 0:
            failed.append((src, text))
        elif verbose and text.strip():
            print(text)
    if failed:
        msg = "\n".join(f"--- {s}\n{t}" for s, t in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    tl = _torch_libdir()
    tmp = lib_path() + ".tmp"
    cmd = ["g++", "-shared", "-o", tmp, *objs, f"-L{tl}", "-lamdhip64", f"-Wl,-rpath,{tl}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, lib_path())
    return lib_path()


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
