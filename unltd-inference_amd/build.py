"""Build recipe for libuq.so (gfx950) and libuq_emu.so (host emulation).

    python unltd-inference_amd/build.py [-v] [-i]   (-i: recompile only stale objects)

libuq.so: every csrc/*.hip plus uq_abi.cpp, uq_gguf.cpp, uq_ops_abi.cpp and uq_layer.cpp, compiled by hipcc for gfx950
  only, -O3, FP contraction off (FMAs are written explicitly), f32
  denormals kept, packed-FP32 instructions disabled. Each source is
  compiled to its own object in parallel (objects under _build/), then
  linked.
libuq_emu.so: csrc/uq_emu.cpp with g++: the kernels' per-lane code run on
  the CPU, used by the CPU test-suite.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(os.path.dirname(HERE), "_build")
LIB = os.path.join(HERE, "libuq.so")
EMU = os.path.join(HERE, "libuq_emu.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # v_dot4_i32_i8 (VOP3P) takes an inline zero accumulator; without this the
    # compiler prefers v_dot4c_i32_i8, whose tied accumulator costs a v_mov per
    # chain start
    "-Xclang", "-target-feature", "-Xclang", "-dot6-insts",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l and "dot6-insts" not in l)  # host pass ignores the device feature
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip"))) + [
        os.path.join(CSRC, f) for f in ("uq_abi.cpp", "uq_gguf.cpp", "uq_ops_abi.cpp", "uq_layer.cpp")]


def _stale(src, obj):
    """An object is stale when it is missing or older than its source or any header of csrc/."""
    if not os.path.exists(obj):
        return True
    deps = [src] + glob.glob(os.path.join(CSRC, "*.h")) + glob.glob(os.path.join(HERE, "..", "include", "*.h"))
    return os.path.getmtime(obj) < max(os.path.getmtime(d) for d in deps)


def build_lib(verbose: bool = False, jobs: int | None = None, incremental: bool = False) -> str:
    """Compiles every source (incremental: only those whose object is stale) and links libuq.so."""
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(OBJ, os.path.basename(s) + ".o") for s in srcs]
    todo = [(s, o) for s, o in zip(srcs, objs) if not incremental or _stale(s, o)]
    jobs = jobs or max(1, min(len(todo), 8, os.cpu_count() or 1))
    with ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda so: _run(["hipcc", *HIPCC_FLAGS, "-x", "hip", "-c", so[0], "-o", so[1]], verbose),
                    todo))
    tmp = LIB + ".tmp"
    _run(["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_emu(verbose: bool = False) -> str:
    tmp = EMU + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
          "-Wall", os.path.join(CSRC, "uq_emu.cpp"), "-o", tmp], verbose)
    os.replace(tmp, EMU)
    return EMU


def build(verbose: bool = False, incremental: bool = False):
    return build_lib(verbose, incremental=incremental), build_emu(verbose)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, incremental="-i" in sys.argv))
