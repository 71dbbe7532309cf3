"""Builds the gfx950 HIP library onnx_amd/liblonnx_hip.so with hipcc.

Usage: python -m onnx_amd.build   (or onnx_amd.build.build())
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "liblonnx_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("LONNX_OFFLOAD_ARCH", "gfx950")
if ARCH != "gfx950":
    # the one-step reciprocal of Erf / GELU and the int32 division seed are proven exact with gfx950's
    # v_rcp_f32 only (tests/native/rcp_check.hip checks every seed on the device)
    raise SystemExit(f"liblonnx_hip is built for gfx950 only (LONNX_OFFLOAD_ARCH={ARCH})")

SOURCES = ["lx_elementwise.hip", "lx_reduce.hip", "lx_softmax.hip", "lx_matmul.hip", "lx_movement.hip", "lx_probe.hip", "lx_api.cpp",
           "lx_pool.cpp", "lx_graph.cpp", "lx_onnx.cpp"]

# -ffp-contract=off: no FMA contraction of separately rounded float ops.
# -fhip-fp32-correctly-rounded-divide-sqrt: IEEE division / sqrt (the reference's semantics).
# -packed-fp32-ops off: no v_pk_*_f32 generation.
# -disable-licm-promotion: LLVM's loop-invariant code motion promotes a store out of a loop whose trip
#   count is one (a template's U = 1 or NV = 1 instance, before the loop is unrolled) and the promoted
#   store loses its nontemporal hint: 44 streaming stores of this library compiled as ordinary stores.
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-disable-licm-promotion",
    "-Wall", "-Wno-unused-function", "-I", os.path.join(HERE, "..", "include"),
]


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC] + COMMON + ["-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC] + COMMON + ["-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=4) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
