"""BACKEND_HIP behind the reference's KernelVTable (guanaco_amd/host).

The CPU tests check the factory conventions of backend.c:5-66 and
test_backend.c: a HIP request without a device is NULL, AUTO falls back to
the CPU backend, dense slots are the CPU kernels, a zeroed Tensor is
rejected.  The GPU test is the drop-in itself: the reference's compiled
engine (oracle/_ref/libref.so: forward(), linear_dispatch, its CPU dense
kernels) runs a whole decode step through the HIP backend's vtable with
device-resident weights, and matches the all-CPU reference."""
import ctypes as C
import os

import numpy as np
import pytest

from oracle import (Q4_K, HostModel, RBackendConfig, RefModel, RTensor, fptr, ref_available,
                    rtensor)
from guanaco_amd import spec as S
from util import rel_l2

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST_SO = os.path.join(ROOT, "guanaco_amd", "libgq_host.so")
BACKEND_AUTO, BACKEND_CPU, BACKEND_HIP = -1, 0, 2


class VTable(C.Structure):  # backend.h:20-39
    _fields_ = [(n, C.c_void_p) for n in ("gemm_f32", "gemm_f32_nn", "rmsnorm", "softmax_inplace",
                                          "silu_inplace", "rope", "residual_add", "elemwise_mul",
                                          "matvec_q4k_f32", "matvec_q6k_f32", "matvec_q8_0_f32")]


@pytest.fixture(scope="module")
def host(ref):
    lib = C.CDLL(HOST_SO)
    lib.backend_create.argtypes = [C.POINTER(RBackendConfig)]
    lib.backend_create.restype = C.c_void_p
    lib.backend_kind.argtypes = [C.c_void_p]
    lib.backend_kernels.argtypes = [C.c_void_p]
    lib.backend_kernels.restype = C.POINTER(VTable)
    lib.backend_destroy.argtypes = [C.c_void_p]
    lib.hip_backend_upload.argtypes = [C.c_void_p, C.POINTER(RTensor)]
    lib.hip_backend_context.argtypes = [C.c_void_p]
    lib.hip_backend_context.restype = C.c_void_p
    return lib


MATVEC = C.CFUNCTYPE(C.c_int, C.POINTER(RTensor), C.POINTER(C.c_float), C.POINTER(C.c_float))


def test_factory_without_device(host, ref):
    import guanaco_amd.hip as H
    if H.device_count() > 0:
        pytest.skip("a GPU is present")
    assert not host.backend_create(C.byref(RBackendConfig(BACKEND_HIP, 2, 0, 0)))
    b = host.backend_create(C.byref(RBackendConfig(BACKEND_AUTO, 2, 0, 0)))
    assert b and host.backend_kind(b) == BACKEND_CPU
    host.backend_destroy(b)


def test_cpu_vtable_conventions(host, ref):
    b = host.backend_create(C.byref(RBackendConfig(BACKEND_CPU, 2, 0, 0)))
    assert b and host.backend_kind(b) == BACKEND_CPU
    vt = host.backend_kernels(b).contents
    assert all(getattr(vt, f) for f, _ in VTable._fields_)
    # zeroed tensor must fail (test_backend.c:71-86)
    W = RTensor()
    x = np.zeros(1, np.float32)
    y = np.zeros(1, np.float32)
    assert MATVEC(vt.matvec_q4k_f32)(C.byref(W), fptr(x), fptr(y)) != 0
    assert MATVEC(vt.matvec_q8_0_f32)(C.byref(W), fptr(x), fptr(y)) != 0
    # gemm KAT through the vtable (test_backend.c:55-77)
    GEMM = C.CFUNCTYPE(None, C.POINTER(RTensor), C.POINTER(RTensor), C.POINTER(RTensor))
    a = np.array([1, 2, 3, 4, 5, 6], np.float32)
    bm = np.array([7, 8, 9, 10, 11, 12], np.float32)
    c = np.zeros(4, np.float32)
    A, B, Cc = rtensor(a, 0, (2, 3)), rtensor(bm, 0, (2, 3)), rtensor(c, 0, (2, 2))
    GEMM(vt.gemm_f32)(C.byref(A), C.byref(B), C.byref(Cc))
    assert np.allclose(c, [50, 68, 122, 167])
    host.backend_destroy(b)


@pytest.mark.gpu
def test_reference_engine_through_hip_vtable(host, ref, orc):
    """Drop-in: reference forward() + HIP vtable with device-resident weights."""
    spec, ms, pre = S.TINY_TEST, 64, 24
    b = host.backend_create(C.byref(RBackendConfig(BACKEND_HIP, 4, 0, spec.n_layers)))
    assert b, "HIP backend unavailable on a GPU box"
    assert host.backend_kind(b) == BACKEND_HIP and host.hip_backend_context(b)
    hm = HostModel(orc, spec, ms)
    cpu = RefModel(ref, hm)
    gpu = RefModel(ref, hm)
    kv = hm.new_kv()
    kv.prefill(orc, spec, pre)
    cpu.load_kv(kv)
    gpu.load_kv(kv)
    # --n-gpu-layers split (loader.c:677-729): first layer GPU-resident only
    n_gpu = 1
    lay = gpu.mw.layers
    for l in range(n_gpu):
        for f in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            assert host.hip_backend_upload(b, getattr(lay[l], f)) == 0
            assert getattr(lay[l], f).contents.device_residency == 1
    assert host.hip_backend_upload(b, gpu.mw.lm_head) == 0
    hip_vt = C.cast(host.backend_kernels(b), C.c_void_p)
    tok_c = tok_g = 9
    for step in range(4):
        tok_c, lc = cpu.forward(tok_c, pre + step)
        out = ref.lib.forward(C.byref(gpu.mw), gpu.kv, gpu.scratch, (C.c_int * 1)(tok_g), 1,
                              pre + step, hip_vt)
        lg = np.ctypeslib.as_array(C.cast(out.contents.data, C.POINTER(C.c_float)),
                                   shape=(spec.vocab,)).copy()
        tok_g = int(ref.lib.sample_greedy(fptr(lg), spec.vocab))
        assert rel_l2(lg, lc) < 1e-3 and tok_g == tok_c, step
    cpu.close()
    gpu.close()
    host.backend_destroy(b)


@pytest.mark.gpu
def test_wide_ff_through_hip_vtable_and_bound_decode(host, ref, orc):
    """ff = 28672 (down rows of 28672 columns, Q6_K and Q4_K; the
    reference's matvec takes any cols % 256, quant_matvec_q4_k.c:143-158):
    every weight device-resident, the reference's forward() through the HIP
    vtable (linear_dispatch, engine.c:119-152) and the device decode of the
    bound model (fused SwiGLU and residual launches at that width) both
    match the all-CPU reference."""
    import guanaco_amd.hip as H
    from oracle import RModelWeights
    spec, ms, pre = S.WIDE_FF_TEST, 32, 9
    b = host.backend_create(C.byref(RBackendConfig(BACKEND_HIP, 4, 0, spec.n_layers)))
    assert b, "HIP backend unavailable on a GPU box"
    host.hip_backend_bind_model.argtypes = [C.c_void_p, C.POINTER(RModelWeights), C.c_void_p]
    hm = HostModel(orc, spec, ms)
    cpu, gpu = RefModel(ref, hm), RefModel(ref, hm)
    kv = hm.new_kv()
    kv.prefill(orc, spec, pre)
    cpu.load_kv(kv)
    gpu.load_kv(kv)
    for l in range(spec.n_layers):
        for f in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            assert host.hip_backend_upload(b, getattr(gpu.mw.layers[l], f)) == 0
            assert getattr(gpu.mw.layers[l], f).contents.device_residency == 1
    assert gpu.mw.layers[0].w_down.contents.shape[1] == 28672
    assert host.hip_backend_upload(b, gpu.mw.lm_head) == 0
    hip_vt = C.cast(host.backend_kernels(b), C.c_void_p)
    tok_c = tok_g = 5
    for step in range(2):
        tok_c, lc = cpu.forward(tok_c, pre + step)
        out = ref.lib.forward(C.byref(gpu.mw), gpu.kv, gpu.scratch, (C.c_int * 1)(tok_g), 1,
                              pre + step, hip_vt)
        lg = np.ctypeslib.as_array(C.cast(out.contents.data, C.POINTER(C.c_float)),
                                   shape=(spec.vocab,)).copy()
        tok_g = int(ref.lib.sample_greedy(fptr(lg), spec.vocab))
        assert rel_l2(lg, lc) < 1e-3 and tok_g == tok_c, step
    # the bound model decodes the next step on the device from the same cache
    assert host.hip_backend_bind_model(b, C.byref(gpu.mw), gpu.kv) == 0
    t_c, lc = cpu.forward(tok_c, pre + 2)
    ld = np.empty(spec.vocab, np.float32)
    t_d = H.lib.gq_hip_forward_token(host.hip_backend_context(b), tok_c, pre + 2,
                                     ld.ctypes.data_as(C.POINTER(C.c_float)), None)
    assert rel_l2(ld, lc) < 1e-3 and t_d == t_c
    cpu.close()
    gpu.close()
    host.backend_destroy(b)


@pytest.mark.gpu
def test_bind_model_and_gpu_prefill_slot(host, ref, orc):
    """The whole model bound from the reference's own ModelWeights
    (hip_backend_bind_model) and the gpu_prefill slot (hip_backend_prefill,
    gpu_prefill.h:13-20): the prompt runs on the device, its K/V rows land
    in the reference's host cache, and the reference's CPU forward() decodes
    the next token from that cache.  Against the all-CPU reference (its
    T-token forward() for the prompt, engine.c:559-595): the bf16 prefill
    tolerance (3e-2 relative L2) and the same greedy token; the device
    decode through the bound model likewise."""
    import guanaco_amd.hip as H
    from oracle import RModelWeights
    spec, ms, n = S.TINY_TEST, 64, 20
    b = host.backend_create(C.byref(RBackendConfig(BACKEND_HIP, 4, 0, spec.n_layers)))
    assert b, "HIP backend unavailable on a GPU box"
    host.hip_backend_bind_model.argtypes = [C.c_void_p, C.POINTER(RModelWeights), C.c_void_p]
    host.hip_backend_prefill.argtypes = [C.c_void_p, C.POINTER(RModelWeights), C.c_void_p, C.c_void_p,
                                         C.POINTER(C.c_int), C.c_int, C.c_int]
    hm = HostModel(orc, spec, ms)
    cpu, gpu = RefModel(ref, hm), RefModel(ref, hm)
    for l in range(spec.n_layers):
        for f in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            assert host.hip_backend_upload(b, getattr(gpu.mw.layers[l], f)) == 0
    assert host.hip_backend_bind_model(b, C.byref(gpu.mw), gpu.kv) == 0
    toks = np.random.default_rng(7).integers(0, spec.vocab, n).astype(np.int32)
    prompt = (C.c_int * (n - 1))(*[int(t) for t in toks[:-1]])
    ref.lib.forward(C.byref(cpu.mw), cpu.kv, cpu.scratch, prompt, n - 1, 0, ref.vtable)
    t_cpu, lc = cpu.forward(int(toks[-1]), n - 1)
    assert host.hip_backend_prefill(b, C.byref(gpu.mw), gpu.kv, gpu.scratch, prompt, n - 1, 0) == 0
    for l in range(spec.n_layers):
        for w in ("k", "v"):
            hk = gpu.slab(w, l).reshape(spec.n_kv_heads, ms, spec.head_dim)[:, :n - 1]
            ck = cpu.slab(w, l).reshape(spec.n_kv_heads, ms, spec.head_dim)[:, :n - 1]
            assert rel_l2(hk, ck) < 3e-2, (l, w)
    t_g, lg = gpu.forward(int(toks[-1]), n - 1)  # the reference's CPU decode on the filled cache
    assert rel_l2(lg, lc) < 3e-2 and t_g == t_cpu
    ctx = host.hip_backend_context(b)
    ld = np.empty(spec.vocab, np.float32)
    t_d = H.lib.gq_hip_forward_token(ctx, int(toks[-1]), n - 1, ld.ctypes.data_as(C.POINTER(C.c_float)), None)
    assert rel_l2(ld, lc) < 3e-2 and t_d == t_cpu
    cpu.close()
    gpu.close()
    host.backend_destroy(b)


@pytest.mark.gpu
def test_n_gpu_layers_split(host, ref, orc):
    """The --n-gpu-layers split (loader.c:672-729, engine.c:314-350): layer 0
    runs on the device through the per-layer hook (gq_hip_transformer_layer:
    host hidden state in and out, its new K/V row written back into the
    reference's host cache), layer 1 through the reference's own CPU
    transformer_layer on that same KVCache.  Against both layers on the CPU:
    each layer's hidden state within the decode tolerance (1e-3 relative L2)
    and the host cache's new rows alike."""
    import guanaco_amd.hip as H
    from oracle import F32, RModelWeights, rtensor
    spec, ms, pre = S.TINY_TEST, 64, 24
    b = host.backend_create(C.byref(RBackendConfig(BACKEND_HIP, 4, 0, spec.n_layers)))
    assert b, "HIP backend unavailable on a GPU box"
    host.hip_backend_bind_model.argtypes = [C.c_void_p, C.POINTER(RModelWeights), C.c_void_p]
    ref.lib.kv_cache_head_stride.argtypes = [C.c_void_p]
    hm = HostModel(orc, spec, ms)
    cpu, mix = RefModel(ref, hm), RefModel(ref, hm)
    kv = hm.new_kv()
    kv.prefill(orc, spec, pre)
    cpu.load_kv(kv)
    mix.load_kv(kv)
    for l in range(spec.n_layers):
        for f in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            assert host.hip_backend_upload(b, getattr(mix.mw.layers[l], f)) == 0
    assert host.hip_backend_bind_model(b, C.byref(mix.mw), mix.kv) == 0  # device cache = host prefix
    ctx = host.hip_backend_context(b)
    h0 = orc.synth_normal(5, spec.hidden)

    def cpu_layer(m, h, l):
        ref.lib.scratch_reset(m.scratch)
        t = rtensor(h, F32, (1, spec.hidden))
        ref.lib.transformer_layer(C.byref(t), C.byref(m.mw.layers[l]), m.kv, l, pre, m.scratch,
                                  C.byref(m.mw.config), ref.vtable)

    hc = [h0.copy()]
    for l in range(spec.n_layers):
        h = hc[-1].copy()
        cpu_layer(cpu, h, l)
        hc.append(h)
    hs = h0.copy()
    rc = H.lib.gq_hip_transformer_layer(ctx, 0, pre, hs.ctypes.data_as(C.POINTER(C.c_float)),
                                        C.cast(ref.lib.kv_cache_raw_k(mix.kv, 0), C.POINTER(C.c_float)),
                                        C.cast(ref.lib.kv_cache_raw_v(mix.kv, 0), C.POINTER(C.c_float)),
                                        ref.lib.kv_cache_head_stride(mix.kv))
    assert rc == 0 and rel_l2(hs, hc[1]) < 1e-3
    for w in ("k", "v"):  # the device layer's new row, in the reference's host cache
        row = lambda m: m.slab(w, 0).reshape(spec.n_kv_heads, ms, spec.head_dim)[:, pre]  # noqa: E731
        assert np.abs(row(mix)).sum() > 0 and rel_l2(row(mix), row(cpu)) < 1e-3
    for l in range(1, spec.n_layers):
        cpu_layer(mix, hs, l)
        assert rel_l2(hs, hc[l + 1]) < 1e-3, l
    cpu.close()
    mix.close()
    host.backend_destroy(b)
