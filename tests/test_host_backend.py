"""BACKEND_HIP behind the reference's KernelVTable (guanaco_amd/host), in
the reference built with guanaco_amd/host/reference-hip.patch applied.

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
# the reference with the HIP backend dropped in (oracle/build_ref_hip.sh):
# the patched factory, engine and loader plus hip_backend.c
HOST_SO = os.path.join(ROOT, "oracle", "_ref", "libref_hip.so")
BACKEND_AUTO, BACKEND_CPU, BACKEND_HIP = -1, 0, 2


class VTable(C.Structure):  # backend.h:20-39
    _fields_ = [(n, C.c_void_p) for n in ("gemm_f32", "gemm_f32_nn", "rmsnorm", "softmax_inplace",
                                          "silu_inplace", "rope", "residual_add", "elemwise_mul",
                                          "matvec_q4k_f32", "matvec_q6k_f32", "matvec_q8_0_f32")]


@pytest.fixture(scope="module")
def host(ref):
    if not os.path.exists(HOST_SO):
        pytest.skip("oracle/_ref/libref_hip.so not built (reference sources absent)")
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
    assert host.hip_backend_upload(b, gpu.mw.lm_head) == 0  # the loader's upload with any device layer
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


@pytest.fixture(scope="module")
def ref_hip(ref):
    from oracle import Ref
    if not os.path.exists(HOST_SO):
        pytest.skip("oracle/_ref/libref_hip.so not built")
    r = Ref(threads=4, path=HOST_SO)
    r.lib.hip_upload_weight.argtypes = [C.POINTER(RTensor)]
    r.lib.hip_backend_bind_model.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
    return r


def _logits(out, vocab):
    return np.ctypeslib.as_array(C.cast(out.contents.data, C.POINTER(C.c_float)), shape=(vocab,)).copy()


@pytest.mark.gpu
def test_patched_engine_prompt_then_device_decode(ref, ref_hip, orc, tmp_path):
    """The reference's own engine with the patch: layer 0 device-resident
    through the loader's hook (hip_upload_weight), the model bound, then

    * a 7-token prompt through the patched forward(): T > 1 takes the CPU
      path, whose new rows of the device-resident layer go to the device
      cache (hip_backend_kv_sync, as cuda_sync_kv_cache at engine.c:394-405);
    * decode steps: layer 0 runs on the device (hip_backend_layer, reading
      those prompt rows from the device cache), layer 1 on the CPU;
    * the session saved by kv_cache_save, loaded into a fresh cache by
      kv_cache_load and the model bound again after the restore (the
      generate.c order): the device cache carries the restored prefix.

    Each step's logits within 1e-3 of the all-CPU reference and the same
    greedy token."""
    from oracle import HostModel, RModelWeights
    spec, ms, pre = S.TINY_TEST, 64, 24
    lib = ref_hip.lib
    b = lib.backend_create(C.byref(RBackendConfig(BACKEND_HIP, 4, 0, 1)))
    assert b, "HIP backend unavailable on a GPU box"
    lib.backend_kernels.restype = C.c_void_p
    hip_vt = C.c_void_p(lib.backend_kernels(b))
    hm = HostModel(orc, spec, ms)
    cpu, mix = RefModel(ref, hm), RefModel(ref_hip, hm)
    kv = hm.new_kv()
    kv.prefill(orc, spec, pre)
    cpu.load_kv(kv)
    mix.load_kv(kv)
    for f in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):  # --n-gpu-layers 1
        assert lib.hip_upload_weight(getattr(mix.mw.layers[0], f)) == 0
    lib.hip_layer_ready.argtypes = [C.c_void_p]
    assert lib.hip_layer_ready(C.addressof(mix.mw.layers[0])) == 1
    assert lib.hip_layer_ready(C.addressof(mix.mw.layers[1])) == 0
    assert lib.hip_backend_bind_model(b, C.addressof(mix.mw), mix.kv) == 0
    prompt = np.random.default_rng(3).integers(0, spec.vocab, 7).astype(np.int32)
    pc = (C.c_int * 7)(*[int(t) for t in prompt])
    lc = _logits(ref.lib.forward(C.byref(cpu.mw), cpu.kv, cpu.scratch, pc, 7, pre, ref.vtable), spec.vocab)
    lm = _logits(lib.forward(C.byref(mix.mw), mix.kv, mix.scratch, pc, 7, pre, hip_vt), spec.vocab)
    assert rel_l2(lm, lc) < 1e-3
    tok = int(ref.lib.sample_greedy(fptr(lc), spec.vocab))
    pos = pre + 7
    for step in range(4):
        t_c, lc = cpu.forward(tok, pos)
        lm = _logits(lib.forward(C.byref(mix.mw), mix.kv, mix.scratch, (C.c_int * 1)(tok), 1, pos, hip_vt),
                     spec.vocab)
        t_m = int(ref.lib.sample_greedy(fptr(lm), spec.vocab))
        assert rel_l2(lm, lc) < 1e-3 and t_m == t_c, step
        tok, pos = t_c, pos + 1
    # the session through the reference's files, restored, then bound again
    path = str(tmp_path / "s.lctx")
    assert lib.kv_cache_save(mix.kv, C.byref(mix.mw.config), ms, pos, None, 0, path.encode()) == 0
    rest = RefModel(ref_hip, hm)
    for f in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
        assert lib.hip_upload_weight(getattr(rest.mw.layers[0], f)) == 0
    got = C.c_int(-1)
    assert lib.kv_cache_load(rest.kv, C.byref(rest.mw.config), ms, C.byref(got), None, None, path.encode()) == 0
    assert got.value == pos
    assert lib.hip_backend_bind_model(b, C.addressof(rest.mw), rest.kv) == 0
    for step in range(3):
        t_c, lc = cpu.forward(tok, pos)
        lm = _logits(lib.forward(C.byref(rest.mw), rest.kv, rest.scratch, (C.c_int * 1)(tok), 1, pos, hip_vt),
                     spec.vocab)
        assert rel_l2(lm, lc) < 1e-3 and int(ref.lib.sample_greedy(fptr(lm), spec.vocab)) == t_c, step
        tok, pos = t_c, pos + 1
    cpu.close(), mix.close(), rest.close()
    lib.backend_destroy(b)

