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


def _run(cmd, verbose, what):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed: {what}")


def build(verbose=False):
    """Each source compiles to its own object (in parallel: the translation
    units share no device code, every kernel is launched from its own file),
    then one link makes the library."""
    from concurrent.futures import ThreadPoolExecutor
    build_som(verbose)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    cflags = [f for f in HIPCC_FLAGS if f != "-shared"]
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in srcs]
    jobs = min(len(srcs), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda so: _run([hipcc()] + cflags + ["-c", os.path.join(CSRC, so[0]), "-o", so[1]], verbose,
                                    so[0]), zip(srcs, objs)))
    tmp = LIB + ".tmp"
    _run([hipcc(), "-shared", "-fPIC", "--offload-arch=gfx950"] + objs + ["-o", tmp], verbose, "link")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
