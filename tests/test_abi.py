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


def test_reference_patch_applies_and_builds(tmp_path):
    """The drop-in as a maintainer applies it: guanaco_amd/host/reference-hip.patch
    applies to the reference's src/ tree as it is, and with hip_backend.c /
    .h added the tree compiles with -DUSE_HIP=1 (the HIP backend under
    -Wall -Wextra -Werror) into the engine library and the command-line
    program, which export the factory (backend.h:41-52) and every hook
    hip_backend.h declares."""
    import subprocess
    from oracle import ref_available
    if not ref_available():
        pytest.skip("reference sources / oracle/_ref not present")
    out = tmp_path / "ref_hip"
    r = subprocess.run(["sh", os.path.join(ROOT, "oracle", "build_ref_hip.sh"), str(out)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    src = open(os.path.join(ROOT, "guanaco_amd", "host", "hip_backend.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = sorted(set(re.findall(r"\b(hip_\w+|backend_hip_\w+)\s*\(", src)))
    assert {"hip_backend_upload", "hip_backend_bind_model", "hip_backend_prefill", "hip_layer_ready",
            "hip_backend_layer", "hip_backend_kv_sync", "hip_upload_weight", "hip_backend_whole",
            "hip_backend_prompt", "hip_backend_forward_sample", "hip_backend_host_kv"} <= set(names)
    lib = ctypes.CDLL(str(out / "libref_hip.so"))
    missing = [n for n in names + ["backend_create", "backend_kernels", "backend_destroy", "backend_hip_create",
                                   "forward", "transformer_layer", "gpu_prefill", "kv_cache_load"]
               if not hasattr(lib, n)]
    assert not missing, missing
    patched = {l.split()[1][2:] for l in open(os.path.join(ROOT, "guanaco_amd", "host", "reference-hip.patch"))
               if l.startswith("+++ ")}
    assert {"backend/backend.c", "backend/backend_internal.h", "include/backend.h", "include/tokenizer.h",
            "tokenizer/tokenizer.c", "main.c", "engine/loader.c", "engine/engine.c", "engine/generate.c",
            "engine/chat.c", "engine/gpu_prefill.c"} <= patched


def test_patched_cli_device_switch(tmp_path):
    """--device hip in the patched command line (tokenizer.c:337-343,
    :385-392, :420-433; main.c:14-42): an unknown kind is refused and names
    hip among the kinds; without a GPU the HIP backend request fails with a
    message instead of falling back."""
    import subprocess
    cli = os.path.join(ROOT, "oracle", "_ref", "guanaco_hip")
    if not os.path.exists(cli):
        pytest.skip("oracle/_ref/guanaco_hip not built")
    r = subprocess.run([cli, "--device", "bogus", "--model", "x"], capture_output=True, text=True, cwd=tmp_path)
    assert r.returncode == 1 and "auto|cpu|cuda|hip" in r.stderr
    import guanaco_amd.hip as H
    if H.device_count() > 0:
        pytest.skip("a GPU is present")
    r = subprocess.run([cli, "--device", "hip", "--model", str(tmp_path / "none.gguf")], capture_output=True,
                       text=True, cwd=tmp_path)
    assert "HIP backend requested but unavailable" in r.stderr
