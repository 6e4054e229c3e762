"""The C-ABI library loads and exports every entry point include/gq_hip.h
declares; without a GPU the context factory fails cleanly (NULL), mirroring
the reference's backend factory returning NULL for an unavailable device
(backend.c:27-33, test_backend.c:92-112)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    src = open(os.path.join(ROOT, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(gq_hip_\w+)\s*\(", src)))


def test_every_declared_symbol_is_exported():
    import guanaco_amd.hip as H
    lib = ctypes.CDLL(H.LIB_PATH)
    names = declared("gq_hip.h")
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python mirror binds each of them
    assert sorted(H.EXPORTS) == names


def test_no_device_means_null_context():
    import guanaco_amd.hip as H
    if H.device_count() > 0:
        pytest.skip("a GPU is present")
    assert not H.lib.gq_hip_create(0)
    with pytest.raises(H.HipError):
        H.Context(0)


def test_host_backend_exports(ref):
    """libgq_host.so (the HIP backend behind the reference's KernelVTable)
    exports the reference's factory (backend.h:41-52) and every hook
    guanaco_amd/host/include/hip_backend.h declares.  Its CPU backend is
    resolved from the reference's objects, so libref.so is loaded first."""
    src = open(os.path.join(ROOT, "guanaco_amd", "host", "include", "hip_backend.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = sorted(set(re.findall(r"\b(hip_backend_\w+)\s*\(", src)))
    assert {"hip_backend_upload", "hip_backend_bind_model", "hip_backend_prefill"} <= set(names)
    lib = ctypes.CDLL(os.path.join(ROOT, "guanaco_amd", "libgq_host.so"))
    missing = [n for n in names + ["backend_create", "backend_kernels", "backend_destroy"]
               if not hasattr(lib, n)]
    assert not missing, missing
