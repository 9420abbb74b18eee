"""The C-ABI libraries build, load and export every symbol include/soso_hip.h,
include/soso_hip_bench.h and include/soso_som.h declare; without a device libsoso_hip refuses cleanly
(no compute calls here)."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("soso_hip.h", "soso_hip_bench.h")]


def declared_symbols():
    text = "".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(soso_hip_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_gpudispatch_surface():
    syms = declared_symbols()
    for s in ("soso_hip_create", "soso_hip_matvec", "soso_hip_matmul", "soso_hip_matvec_batch",
              "soso_hip_router_topk", "soso_hip_experts_block", "soso_hip_dtype_supported", "soso_hip_stats"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    from soso_amd import abi
    lib = abi.load()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    # and the ctypes prototypes cover exactly that list
    assert sorted(abi.PROTOTYPES) == declared_symbols()


def test_som_library_exports_every_declared_symbol():
    """libsoso_som.so against include/soso_som.h, and the Python binding's
    prototypes cover exactly that list."""
    from soso_amd import som
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "soso_som.h")).read(), flags=re.S)
    syms = sorted(set(re.findall(r"\b(soso_som_[a-z0-9_]+)\s*\(", text)))
    lib = som.lib()
    assert syms and not [s for s in syms if not hasattr(lib, s)]
    src = open(som.__file__).read()
    assert sorted(set(re.findall(r'"(soso_som_[a-z0-9_]+)"', src))) == syms


def test_null_and_bad_arguments_are_errors_not_crashes():
    from soso_amd import abi
    lib = abi.load()
    assert lib.soso_hip_create(0, 0, None) < 0
    assert lib.soso_hip_available(None) == 0
    assert lib.soso_hip_dtype_supported(None, 3) == 0
    assert lib.soso_hip_matvec(None, b"k", 1, None, 0, 3, 1, 256, None, None) < 0
    assert lib.soso_hip_last_error(None) == b"null handle"


def test_create_without_device_fails_cleanly():
    """In a container with no GPU, create returns an error instead of crashing."""
    from soso_amd import abi
    lib = abi.load()
    h = C.c_void_p()
    rc = lib.soso_hip_create(0, 0, C.byref(h))
    if rc == 0:
        lib.soso_hip_destroy(h)
        pytest.skip("a device is present")
    assert rc < 0 and not h.value


def test_python_view_mirrors_trait_names():
    from soso_amd.dispatch import HipGpu
    for m in ("available", "dtype_soportado", "stats", "matvec", "matmul", "matvec_lote", "router_topk",
              "expertos_bloque"):
        assert callable(getattr(HipGpu, m))
