"""ctypes bindings of the CPU checker (TEST INFRASTRUCTURE ONLY).

``Oracle`` wraps ``oracle/liboracle.so`` (the C restatement of the reference's
CPU arithmetic, ``gq_oracle.c``).  ``Ref`` wraps ``oracle/_ref/libref.so``,
the reference's own CPU path compiled from its sources by ``oracle/Makefile``
(present only where the reference sources were available at build time).
``HostModel`` materialises a synthetic model (``guanaco_amd.spec``) in host
memory and exposes it to both.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg use
this module; the product (``guanaco_amd``) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")

F32, Q8_0, Q4_K, Q6_K = 0, 2, 4, 5
SYNTH_Q4K_ZERO_MEAN = 0x100  # gq_synth.h: the zero-mean Q4_K generator code
_fp = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)


def fptr(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def u8ptr(a):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(_u8p)


class OrcTensor(C.Structure):
    _fields_ = [("dtype", C.c_int), ("rows", C.c_int), ("cols", C.c_int),
                ("data", _u8p), ("bytes", C.c_size_t)]


class OrcModel(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "hidden", "ff", "n_heads", "n_kv_heads",
                                      "head_dim", "vocab", "max_seq")] + [
        ("rope_theta", C.c_float), ("rms_eps", C.c_float)] + [
        (n, C.POINTER(OrcTensor)) for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")] + [
        ("rms_att", C.POINTER(_fp)), ("rms_ffn", C.POINTER(_fp)),
        ("embed", OrcTensor), ("lm_head", OrcTensor), ("rms_final", _fp)]


class OrcKV(C.Structure):
    _fields_ = [("k", _fp), ("v", _fp), ("n_layers", C.c_int), ("n_kv_heads", C.c_int),
                ("head_dim", C.c_int), ("max_seq", C.c_int)]


class Oracle:
    def __init__(self, path=ORACLE_SO, threads=None):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        for n in ("orc_matvec_q4k", "orc_matvec_q6k", "orc_matvec_q8_0"):
            getattr(L, n).argtypes = [_u8p, C.c_size_t, C.c_int, C.c_int, _fp, _fp]
            getattr(L, n).restype = C.c_int
        L.orc_rmsnorm.argtypes = [_fp, _fp, _fp, C.c_int, C.c_float]
        L.orc_dot8.argtypes = [_fp, _fp, C.c_int]
        L.orc_dot8.restype = C.c_float
        L.orc_softmax.argtypes = [_fp, C.c_int]
        L.orc_silu.argtypes = [_fp, C.c_int]
        L.orc_rope.argtypes = [_fp, _fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        L.orc_rope_table.argtypes = [_fp, _fp, C.c_int, C.c_int, C.c_float]
        L.orc_attention.argtypes = [_fp, C.POINTER(OrcKV), C.c_int, C.c_int, C.c_int, _fp]
        L.orc_embed.argtypes = [C.POINTER(OrcTensor), C.c_int, _fp]
        L.orc_argmax.argtypes = [_fp, C.c_int]
        L.orc_kv_append.argtypes = [C.POINTER(OrcKV), C.c_int, C.c_int, _fp, _fp]
        L.orc_layer.argtypes = [C.POINTER(OrcModel), C.POINTER(OrcKV), C.c_int, C.c_int, _fp]
        L.orc_forward_token.argtypes = [C.POINTER(OrcModel), C.POINTER(OrcKV), C.c_int, C.c_int,
                                        _fp, _fp]
        L.orc_lctx_size.argtypes = [C.POINTER(OrcKV), C.c_int]
        L.orc_lctx_size.restype = C.c_size_t
        L.orc_lctx_write.argtypes = [C.POINTER(OrcKV), C.c_int, C.POINTER(C.c_int32), C.c_int,
                                     _u8p, C.c_size_t]
        L.orc_lctx_read.argtypes = [C.POINTER(OrcKV), _u8p, C.c_size_t, C.POINTER(C.c_int),
                                    C.POINTER(C.c_int)]
        for n in ("orc_synth_q4k", "orc_synth_q4k_zm", "orc_synth_q6k", "orc_synth_q8_0"):
            getattr(L, n).argtypes = [C.c_uint64, C.c_int, C.c_int, _u8p]
        L.orc_synth_normal.argtypes = [C.c_uint64, C.c_size_t, _fp]
        L.orc_synth_norm_weight.argtypes = [C.c_uint64, C.c_size_t, _fp]
        L.orc_tensor_seed.argtypes = [C.c_uint64, C.c_int, C.c_int]
        L.orc_tensor_seed.restype = C.c_uint64
        L.orc_synth_kv.argtypes = [C.c_uint64, _fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_set_faithful.argtypes = [C.c_int]
        self.set_threads(threads or min(os.cpu_count() or 1, 16))

    def set_threads(self, n):
        self.lib.orc_set_threads(int(n))
        self.threads = int(n)

    def set_faithful(self, on):
        self.lib.orc_set_faithful(1 if on else 0)

    # ---- synthetic inputs ----
    def tensor_seed(self, model_seed, layer, slot):
        return int(self.lib.orc_tensor_seed(model_seed, layer, slot))

    def synth_quant(self, dtype, seed, rows, cols):
        """Blocks of a generator code: a dtype, or Q4_K | SYNTH_Q4K_ZERO_MEAN."""
        zm = dtype == (Q4_K | SYNTH_Q4K_ZERO_MEAN)
        qk, bb = {Q4_K: (256, 144), Q6_K: (256, 210), Q8_0: (32, 34)}[Q4_K if zm else dtype]
        out = np.empty(rows * (cols // qk) * bb, np.uint8)
        fn = self.lib.orc_synth_q4k_zm if zm else {Q4_K: self.lib.orc_synth_q4k, Q6_K: self.lib.orc_synth_q6k,
                                                   Q8_0: self.lib.orc_synth_q8_0}[dtype]
        fn(seed, rows, cols, u8ptr(out))
        return out

    def synth_normal(self, seed, n):
        out = np.empty(n, np.float32)
        self.lib.orc_synth_normal(seed, n, fptr(out))
        return out

    def synth_norm_weight(self, seed, n, shift=0):
        """(1 + N(0,1)/64) * 2^-shift, exact in fp32."""
        out = np.empty(n, np.float32)
        self.lib.orc_synth_norm_weight(seed, n, fptr(out))
        return np.ldexp(out, -shift).astype(np.float32) if shift else out

    # ---- kernels ----
    def matvec(self, dtype, w, rows, cols, x, nbytes=None):
        y = np.zeros(rows, np.float32)
        fn = {Q4_K: self.lib.orc_matvec_q4k, Q6_K: self.lib.orc_matvec_q6k,
              Q8_0: self.lib.orc_matvec_q8_0}[dtype]
        rc = fn(u8ptr(w), w.nbytes if nbytes is None else nbytes, rows, cols,
                fptr(np.ascontiguousarray(x, np.float32)), fptr(y))
        if rc:
            raise ValueError(f"oracle matvec rc={rc}")
        return y

    def rmsnorm(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self.lib.orc_rmsnorm(fptr(x), fptr(w) if w is not None else None, fptr(out), x.size, eps)
        return out

    def rope_table(self, head_dim, pos, theta):
        c = np.empty(head_dim // 2, np.float32)
        s = np.empty(head_dim // 2, np.float32)
        self.lib.orc_rope_table(fptr(c), fptr(s), head_dim, pos, theta)
        return c, s

    def rope(self, q, k, n_heads, n_kv, head_dim, pos, theta):
        q = np.array(q, np.float32)
        k = np.array(k, np.float32)
        self.lib.orc_rope(fptr(q), fptr(k), n_heads, n_kv, head_dim, pos, theta)
        return q, k

    def attention(self, q, kv, layer, n_heads, pos):
        out = np.empty(n_heads * kv.head_dim, np.float32)
        self.lib.orc_attention(fptr(np.ascontiguousarray(q, np.float32)), C.byref(kv.s), layer,
                               n_heads, pos, fptr(out))
        return out

    def argmax(self, x):
        return int(self.lib.orc_argmax(fptr(np.ascontiguousarray(x, np.float32)), x.size))


class HostKV:
    """fp32 K/V slabs [layer][kv_head][max_seq][head_dim] (kv_cache.c:25-32)."""

    def __init__(self, n_layers, n_kv_heads, head_dim, max_seq):
        n = n_layers * n_kv_heads * max_seq * head_dim
        self.k = np.zeros(n, np.float32)
        self.v = np.zeros(n, np.float32)
        self.n_layers, self.n_kv_heads, self.head_dim, self.max_seq = (
            n_layers, n_kv_heads, head_dim, max_seq)
        self.s = OrcKV(fptr(self.k), fptr(self.v), n_layers, n_kv_heads, head_dim, max_seq)

    def view(self, which="k"):
        a = self.k if which == "k" else self.v
        return a.reshape(self.n_layers, self.n_kv_heads, self.max_seq, self.head_dim)

    def prefill(self, orc, spec, n_pos):
        """Seeded N(0,1) history at positions 0..n_pos-1 (gq_kv_index order)."""
        for arr, slot in ((self.k, 13), (self.v, 14)):
            orc.lib.orc_synth_kv(orc.tensor_seed(spec.seed, -1, slot), fptr(arr), self.n_layers,
                                 self.n_kv_heads, self.head_dim, self.max_seq, n_pos)


class HostModel:
    """Synthetic model in host memory, visible to the oracle and the reference."""

    def __init__(self, orc: Oracle, spec, max_seq):
        self.spec, self.orc, self.max_seq = spec, orc, max_seq
        s = spec
        self.w = {}
        keep = []

        def qt(dtype, seed, rows, cols):
            data = orc.synth_quant(s.gen(dtype), seed, rows, cols)
            keep.append(data)
            return data, OrcTensor(dtype, rows, cols, u8ptr(data), data.nbytes)

        L = s.n_layers
        arrs = {k: (OrcTensor * L)() for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")}
        self.layer_w = [dict() for _ in range(L)]
        self.rms_att = [None] * L
        self.rms_ffn = [None] * L
        slots = dict(wq=0, wk=1, wv=2, wo=3, wg=4, wu=5, wd=6)
        for l in range(L):
            dts = s.dtypes(l)
            for k, slot in slots.items():
                rows, cols = s.shape(k)
                data, t = qt(dts[k], orc.tensor_seed(s.seed, l, slot), rows, cols)
                arrs[k][l] = t
                self.layer_w[l][k] = (dts[k], data)
            self.rms_att[l] = orc.synth_norm_weight(orc.tensor_seed(s.seed, l, 7), s.hidden, s.norm_shift)
            self.rms_ffn[l] = orc.synth_norm_weight(orc.tensor_seed(s.seed, l, 8), s.hidden, s.norm_shift)
        self.embed, embed_t = qt(s.embed_dtype, orc.tensor_seed(s.seed, -1, 10), s.vocab, s.hidden)
        self.lm_head, lm_t = qt(s.lm_head_dtype, orc.tensor_seed(s.seed, -1, 11), s.vocab,
                                s.hidden)
        self.rms_final = orc.synth_norm_weight(orc.tensor_seed(s.seed, -1, 12), s.hidden, s.norm_shift)
        att_p = (_fp * L)(*[fptr(a) for a in self.rms_att])
        ffn_p = (_fp * L)(*[fptr(a) for a in self.rms_ffn])
        self._keep = (keep, arrs, att_p, ffn_p)
        self.s = OrcModel(L, s.hidden, s.ff, s.n_heads, s.n_kv_heads, s.head_dim, s.vocab,
                          max_seq, s.rope_theta, s.rms_eps,
                          *[C.cast(arrs[k], C.POINTER(OrcTensor))
                            for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")],
                          C.cast(att_p, C.POINTER(_fp)), C.cast(ffn_p, C.POINTER(_fp)),
                          embed_t, lm_t, fptr(self.rms_final))

    def new_kv(self):
        s = self.spec
        return HostKV(s.n_layers, s.n_kv_heads, s.head_dim, self.max_seq)

    def forward(self, kv, token, pos, want_hidden=False):
        s = self.spec
        logits = np.empty(s.vocab, np.float32)
        hid = np.empty(s.n_layers * s.hidden, np.float32) if want_hidden else None
        tok = self.orc.lib.orc_forward_token(C.byref(self.s), C.byref(kv.s), token, pos,
                                            fptr(logits), fptr(hid) if want_hidden else None)
        return tok, logits, (hid.reshape(s.n_layers, s.hidden) if want_hidden else None)


# --------------------------------------------------------------------------
# The reference itself (oracle/_ref/libref.so), through its own C interface.

class RTensor(C.Structure):  # types.h:51-62
    _fields_ = [("data", C.c_void_p), ("shape", C.c_int * 4), ("stride", C.c_int * 4),
                ("ndim", C.c_int), ("dtype", C.c_int), ("ggml_type", C.c_uint32),
                ("byte_size", C.c_size_t), ("device_residency", C.c_int),
                ("d_data", C.c_void_p)]


class RModelConfig(C.Structure):  # types.h:110-123
    _fields_ = [(n, C.c_int) for n in ("hidden_dim", "n_heads", "n_kv_heads", "head_dim",
                                      "n_layers", "vocab_size", "bos_token_id", "eos_token_id",
                                      "ff_dim", "max_seq_len")] + [
        ("vocab_strings", C.c_void_p), ("vocab_scores", C.c_void_p)]


class RLayerWeights(C.Structure):  # types.h:127-137
    _fields_ = [(n, C.POINTER(RTensor)) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up",
                                                  "w_down", "rms_att", "rms_ffn")]


class RModelWeights(C.Structure):  # types.h:141-147
    _fields_ = [("config", RModelConfig), ("layers", C.POINTER(RLayerWeights)),
                ("embedding", C.POINTER(RTensor)), ("rms_final", C.POINTER(RTensor)),
                ("lm_head", C.POINTER(RTensor))]


class RBackendConfig(C.Structure):  # backend.h:41-46
    _fields_ = [("kind", C.c_int), ("threads", C.c_int), ("device_id", C.c_int),
                ("n_gpu_layers", C.c_int)]


def rtensor(data, dtype, shape, byte_size=None):
    t = RTensor()
    t.data = data.ctypes.data
    t.ndim = len(shape)
    for i, n in enumerate(shape):
        t.shape[i] = n
    st = 1
    for i in range(len(shape) - 1, -1, -1):
        t.stride[i] = st
        st *= shape[i]
    t.dtype = dtype
    t.byte_size = data.nbytes if byte_size is None else byte_size
    return t


def ref_available():
    return os.path.exists(REF_SO)


class Ref:
    """The reference CPU path (compiled, unmodified) — pins the oracle."""

    def __init__(self, threads=8, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        # only the unmodified reference goes into the global namespace
        L = self.lib = C.CDLL(path, mode=C.RTLD_GLOBAL if path == REF_SO else C.RTLD_LOCAL)
        for n in ("matvec_q4k_f32", "matvec_q6k_f32", "matvec_q8_0_f32"):
            getattr(L, n).argtypes = [C.POINTER(RTensor), _fp, _fp]
            getattr(L, n).restype = C.c_int
        L.backend_create.argtypes = [C.POINTER(RBackendConfig)]
        L.backend_create.restype = C.c_void_p
        L.backend_kernels.argtypes = [C.c_void_p]
        L.backend_kernels.restype = C.c_void_p
        L.backend_destroy.argtypes = [C.c_void_p]
        L.arena_create.argtypes = [C.c_size_t]
        L.arena_create.restype = C.c_void_p
        L.arena_destroy.argtypes = [C.c_void_p]
        L.scratch_create.argtypes = [C.c_size_t]
        L.scratch_create.restype = C.c_void_p
        L.scratch_destroy.argtypes = [C.c_void_p]
        L.kv_cache_create.argtypes = [C.c_void_p, C.POINTER(RModelConfig), C.c_int]
        L.kv_cache_create.restype = C.c_void_p
        L.kv_cache_raw_k.argtypes = [C.c_void_p, C.c_int]
        L.kv_cache_raw_k.restype = C.c_void_p
        L.kv_cache_raw_v.argtypes = [C.c_void_p, C.c_int]
        L.kv_cache_raw_v.restype = C.c_void_p
        L.kv_cache_append.argtypes = [C.c_void_p, C.c_int, C.POINTER(RTensor),
                                      C.POINTER(RTensor), C.c_int]
        L.kv_cache_append.restype = C.c_int
        L.kv_cache_save.argtypes = [C.c_void_p, C.POINTER(RModelConfig), C.c_int, C.c_int,
                                    C.POINTER(C.c_int), C.c_int, C.c_char_p]
        L.kv_cache_save.restype = C.c_int
        L.kv_cache_load.argtypes = [C.c_void_p, C.POINTER(RModelConfig), C.c_int,
                                    C.POINTER(C.c_int), C.POINTER(C.POINTER(C.c_int)),
                                    C.POINTER(C.c_int), C.c_char_p]
        L.kv_cache_load.restype = C.c_int
        L.prompt_cache_save.argtypes = [C.c_void_p, C.POINTER(RModelConfig), C.c_int, C.c_int, C.c_char_p]
        L.prompt_cache_save.restype = C.c_int
        L.prompt_cache_load.argtypes = [C.c_void_p, C.POINTER(RModelConfig), C.c_int,
                                        C.POINTER(C.c_int), C.c_char_p]
        L.prompt_cache_load.restype = C.c_int
        L.forward.argtypes = [C.POINTER(RModelWeights), C.c_void_p, C.c_void_p,
                              C.POINTER(C.c_int), C.c_int, C.c_int, C.c_void_p]
        L.forward.restype = C.POINTER(RTensor)
        L.transformer_layer.argtypes = [C.POINTER(RTensor), C.POINTER(RLayerWeights), C.c_void_p,
                                        C.c_int, C.c_int, C.c_void_p, C.POINTER(RModelConfig),
                                        C.c_void_p]
        L.scratch_reset.argtypes = [C.c_void_p]
        L.sample_greedy.argtypes = [_fp, C.c_int]
        L.sample_greedy.restype = C.c_int
        L.rope.argtypes = [C.POINTER(RTensor), C.POINTER(RTensor), C.c_int, C.c_int]
        L.cpu_rmsnorm.argtypes = [C.POINTER(RTensor), C.POINTER(RTensor), C.POINTER(RTensor),
                                  C.c_float]
        L.softmax_inplace.argtypes = [C.POINTER(RTensor), C.c_int]
        L.silu_inplace.argtypes = [C.POINTER(RTensor)]
        cfg = RBackendConfig(0, threads, 0, 0)  # BACKEND_CPU
        self.backend = L.backend_create(C.byref(cfg))
        self.vtable = L.backend_kernels(self.backend)

    def matvec(self, dtype, w, rows, cols, x, nbytes=None):
        t = rtensor(w, dtype, (rows, cols), nbytes)
        y = np.zeros(rows, np.float32)
        fn = {Q4_K: self.lib.matvec_q4k_f32, Q6_K: self.lib.matvec_q6k_f32,
              Q8_0: self.lib.matvec_q8_0_f32}[dtype]
        rc = fn(C.byref(t), fptr(np.ascontiguousarray(x, np.float32)), fptr(y))
        if rc:
            raise ValueError(f"reference matvec rc={rc}")
        return y


class RefModel:
    """The HostModel's buffers wrapped as the reference's ModelWeights, with
    the reference's own KV cache, scratch and forward()."""

    def __init__(self, ref: Ref, hm: HostModel):
        s = hm.spec
        self.ref, self.hm, self.spec = ref, hm, s
        keep = []

        def T(data, dtype, shape):
            t = rtensor(data, dtype, shape)
            keep.append(t)
            return C.pointer(t)

        L = s.n_layers
        layers = (RLayerWeights * L)()
        for l in range(L):
            lw = hm.layer_w[l]
            args = [T(lw[k][1], lw[k][0], s.shape(k)) for k in
                    ("wq", "wk", "wv", "wo", "wg", "wu", "wd")]
            args += [T(hm.rms_att[l], F32, (s.hidden,)), T(hm.rms_ffn[l], F32, (s.hidden,))]
            layers[l] = RLayerWeights(*args)
        cfg = RModelConfig(s.hidden, s.n_heads, s.n_kv_heads, s.head_dim, L, s.vocab, 1, 2,
                           s.ff, hm.max_seq, None, None)
        self.mw = RModelWeights(cfg, C.cast(layers, C.POINTER(RLayerWeights)),
                                T(hm.embed, s.embed_dtype, (s.vocab, s.hidden)),
                                T(hm.rms_final, F32, (s.hidden,)),
                                T(hm.lm_head, s.lm_head_dtype, (s.vocab, s.hidden)))
        self._keep = (keep, layers)
        kv_bytes = 2 * L * s.n_kv_heads * hm.max_seq * s.head_dim * 4
        self.arena = ref.lib.arena_create(kv_bytes + (64 << 20))
        self.scratch = ref.lib.scratch_create(512 << 20)  # generate.c:132
        self.kv = ref.lib.kv_cache_create(self.arena, C.byref(self.mw.config), hm.max_seq)
        if not self.kv:
            raise MemoryError("reference kv_cache_create failed")

    def slab(self, which, layer):
        s = self.spec
        n = s.n_kv_heads * self.hm.max_seq * s.head_dim
        ptr = (self.ref.lib.kv_cache_raw_k if which == "k" else self.ref.lib.kv_cache_raw_v)(
            self.kv, layer)
        return np.ctypeslib.as_array(C.cast(ptr, _fp), shape=(n,))

    def load_kv(self, hkv: HostKV):
        s = self.spec
        n = s.n_kv_heads * self.hm.max_seq * s.head_dim
        for l in range(s.n_layers):
            self.slab("k", l)[:] = hkv.k[l * n:(l + 1) * n]
            self.slab("v", l)[:] = hkv.v[l * n:(l + 1) * n]

    def forward(self, token, pos):
        tok = (C.c_int * 1)(token)
        out = self.ref.lib.forward(C.byref(self.mw), self.kv, self.scratch, tok, 1, pos,
                                   self.ref.vtable)
        logits = np.ctypeslib.as_array(C.cast(out.contents.data, _fp),
                                       shape=(self.spec.vocab,)).copy()
        return int(self.ref.lib.sample_greedy(fptr(logits), self.spec.vocab)), logits

    def close(self):
        self.ref.lib.scratch_destroy(self.scratch)
        self.ref.lib.arena_destroy(self.arena)
