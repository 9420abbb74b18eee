"""Builds libsoso_hip.so (HIP kernels + C ABI) for gfx950 and libsoso_som.so
(the host-side .som reader), in-tree.

Called by __graft_entry__.build(); also runnable as `python -m soso_amd.build`.
hipcc cross-compiles for gfx950 without a GPU.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libsoso_hip.so")
SOURCES = ["runtime.hip", "k_matvec.hip", "k_moe.hip", "k_synth.hip", "k_decode.hip", "k_mfma.hip", "k_gdn.hip"]

# Packed FP32 VALU ops are disabled for all device code; hipcc's host pass
# warns that it does not know the feature, which is harmless.
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared", "--offload-arch=gfx950",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument", "-Wno-unused-result",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


SOM_LIB = os.path.join(HERE, "libsoso_som.so")
SOM_SOURCES = ["som.cpp"]  # host-only: the .som reader (include/soso_som.h)


def build_som(verbose=False):
    """libsoso_som.so: host C++ (g++), no GPU code."""
    tmp = SOM_LIB + ".tmp"
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall"] + \
        [os.path.join(CSRC, s) for s in SOM_SOURCES] + ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("g++ failed building libsoso_som.so")
    os.replace(tmp, SOM_LIB)
    return SOM_LIB


def build(verbose=False):
    build_som(verbose)
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    tmp = LIB + ".tmp"
    cmd = [hipcc()] + HIPCC_FLAGS + srcs + ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building libsoso_hip.so")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
