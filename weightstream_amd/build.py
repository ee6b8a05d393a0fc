"""Build the gfx950 libraries in-tree with hipcc.

    python -m weightstream_amd.build

Objects go to weightstream_amd/_build/. Two libraries share every object but
the one that fixes the math mode (csrc/math_mode.hip):
  weightstream_amd/libweightstream_hip.so         WS_MATH_EXACT (the product)
  weightstream_amd/libweightstream_hip_native.so  WS_MATH_NATIVE (CDNA4 scaled MFMA)
weightstream_amd._lib loads them.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libweightstream_hip.so")
LIB_NATIVE = os.path.join(PKG, "libweightstream_hip_native.so")

SOURCES = ["common.hip", "pack.hip", "gemm.hip", "gemm_line.hip", "moe_route.hip", "moe_decode.hip", "moe_grouped.hip",
           "moe_shared.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # f32 arithmetic of the exact paths (routing, quantisation) must not be
    # contracted into FMAs; MFMA accumulation is unaffected
    "-ffp-contract=off",
    # packed FP32 VALU ops are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-I" + os.path.join(ROOT, "include"),
]


def hipcc():
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def _compile(job):
    src, obj, extra = job
    cmd = [hipcc()] + HIPCC_FLAGS + extra + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s%s" % (src, r.stdout, r.stderr))
    return obj


def _link(objs, lib):
    tmp = lib + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n%s%s" % (r.stdout, r.stderr))
    os.replace(tmp, lib)


def build(verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    o = lambda name: os.path.join(BUILD, name)
    jobs = [(s, o(os.path.splitext(s)[0] + ".o"), []) for s in SOURCES]
    jobs += [("math_mode.hip", o("math_mode.o"), []),
             ("math_mode.hip", o("math_mode_native.o"), ["-DWS_NATIVE_MATH"])]
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        objs = list(ex.map(_compile, jobs))
    shared = objs[:len(SOURCES)]
    _link(shared + [o("math_mode.o")], LIB)
    _link(shared + [o("math_mode_native.o")], LIB_NATIVE)
    if verbose:
        print("built", LIB, "and", LIB_NATIVE)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
