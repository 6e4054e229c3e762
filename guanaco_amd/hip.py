"""ctypes mirror of the C ABI in include/gq_hip.h (libgq_hip.so).

The library is loaded from this package directory; importing this module on
a machine without the built library raises ImportError, and every call that
needs a GPU raises ``HipError`` when the device or the call fails — there is
no CPU fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import spec as S

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgq_hip.so")

_fp = C.POINTER(C.c_float)
_vp = C.c_void_p


class HipError(RuntimeError):
    pass


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
    L = C.CDLL(LIB_PATH)
    sig = {
        "gq_hip_device_count": (C.c_int, []),
        "gq_hip_create": (_vp, [C.c_int]),
        "gq_hip_destroy": (None, [_vp]),
        "gq_hip_last_error": (C.c_char_p, [_vp]),
        "gq_hip_sync": (C.c_int, [_vp]),
        "gq_hip_device_info": (C.c_int, [_vp, C.POINTER(C.c_int), C.c_char_p, C.c_int]),
        "gq_hip_upload_weight": (_vp, [_vp, _vp, C.c_size_t]),
        "gq_hip_mem_info": (C.c_int, [C.c_int, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
        "gq_hip_malloc": (_vp, [_vp, C.c_size_t]),
        "gq_hip_free": (None, [_vp, _vp]),
        "gq_hip_h2d": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
        "gq_hip_d2h": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
        "gq_hip_synth_quant": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, C.c_uint64]),
        "gq_hip_synth_normal": (C.c_int, [_vp, _vp, C.c_size_t, C.c_uint64]),
        "gq_hip_synth_norm_weight": (C.c_int, [_vp, _vp, C.c_size_t, C.c_uint64]),
        "gq_hip_matvec": (C.c_int, [_vp, C.c_int, _vp, C.c_int, C.c_int, C.c_size_t, _fp, _fp]),
        "gq_hip_matvec_dev": (C.c_int, [_vp, C.c_int, _vp, C.c_int, C.c_int, _vp, _vp]),
        "gq_hip_matvec_norm_dev": (C.c_int, [_vp, C.c_int, _vp, C.c_int, C.c_int, _vp, _vp, C.c_float, _vp]),
        "gq_hip_kv_init": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]),
        "gq_hip_kv_k": (_vp, [_vp, C.c_int]),
        "gq_hip_kv_v": (_vp, [_vp, C.c_int]),
        "gq_hip_kv_append": (C.c_int, [_vp, C.c_int, C.c_int, _fp, _fp]),
        "gq_hip_kv_read_layer": (C.c_int, [_vp, C.c_int, _fp, _fp]),
        "gq_hip_kv_write_layer": (C.c_int, [_vp, C.c_int, _fp, _fp]),
        "gq_hip_kv_sync": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _fp, _fp, C.c_int, C.c_int]),
        "gq_hip_kv_prefill_synth": (C.c_int, [_vp, C.c_uint64, C.c_uint64, C.c_int]),
        "gq_hip_kv_fetch": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _fp, _fp, C.c_int, C.c_int]),
        "gq_hip_lctx_save": (C.c_int, [_vp, C.c_char_p, C.c_int, C.POINTER(C.c_int32), C.c_int]),
        "gq_hip_prompt_cache_save": (C.c_int, [_vp, C.c_int, C.c_char_p]),
        "gq_hip_prompt_cache_load": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_int)]),
        "gq_hip_lctx_load": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_int),
                                       C.POINTER(C.POINTER(C.c_int32)), C.POINTER(C.c_int)]),
        "gq_hip_lctx_restore_image": (C.c_int, [_vp, _vp, C.c_size_t, C.POINTER(C.c_int),
                                                C.POINTER(C.c_float)]),
        "gq_hip_host_alloc_pinned": (_vp, [C.c_size_t]),
        "gq_hip_host_free_pinned": (None, [_vp]),
        "gq_hip_model_bind": (C.c_int, [_vp, _vp]),
        "gq_hip_bound_layers": (C.c_int, [_vp, _vp]),
        "gq_hip_set_prefill_mode": (C.c_int, [_vp, C.c_int]),
        "gq_hip_decode_layer_dev": (C.c_int, [_vp, C.c_int, C.c_int, _vp]),
        "gq_hip_transformer_layer": (C.c_int, [_vp, C.c_int, C.c_int, _fp, _fp, _fp, C.c_int]),
        "gq_hip_forward_token": (C.c_int, [_vp, C.c_int, C.c_int, _fp, _fp]),
        "gq_hip_sample_dev": (C.c_int, [_vp, _vp, C.c_int, C.c_float, C.c_int, C.c_float, C.c_int]),
        "gq_hip_forward_sample": (C.c_int, [_vp, C.c_int, C.c_int, C.c_float, C.c_int, C.c_float, C.c_int]),
        "gq_hip_decode_loop": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int,
                                         C.POINTER(C.c_int32), C.POINTER(C.c_float)]),
        "gq_hip_profile_step": (C.c_int, [_vp, C.c_int, C.c_int, C.POINTER(C.c_double),
                                          C.POINTER(C.c_int), C.POINTER(C.c_double)]),
        "gq_hip_time_matvec": (C.c_float, [_vp, C.c_int, C.POINTER(_vp), C.c_int, C.c_int,
                                           C.c_int, _vp, _vp, C.c_int]),
        "gq_hip_set_matvec_path": (C.c_int, [C.c_int]),
        "gq_hip_time_op": (C.c_float, [_vp, C.c_int, C.c_int, C.c_int]),
        "gq_hip_time_attention": (C.c_float, [_vp, C.c_int, C.c_int, _vp, _vp, C.c_int]),
        "gq_hip_rmsnorm_dev": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, C.c_float]),
        "gq_hip_rope_append_dev": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp]),
        "gq_hip_attention_dev": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp]),
        "gq_hip_attention_dev_noalloc": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp]),
        "gq_hip_qkv_rope_dev": (C.c_int, [_vp, C.c_int, C.c_int, _vp, _vp, C.c_int]),
        "gq_hip_embed_dev": (C.c_int, [_vp, C.c_int, _vp, C.c_int, C.c_int, _vp]),
        "gq_hip_argmax_dev": (C.c_int, [_vp, _vp, C.c_int, _vp]),
        "gq_hip_silu_mul_dev": (C.c_int, [_vp, _vp, _vp, C.c_int]),
        "gq_hip_copy_dev": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
        "gq_hip_time_read": (C.c_float, [_vp, _vp, C.c_size_t, C.c_size_t, C.c_int, C.c_int]),
        "gq_hip_time_prefill_gemm": (C.c_float, [_vp, C.c_int, _vp, C.c_int, C.c_int, _vp, C.c_int, _vp, C.c_int]),
        "gq_hip_prefill_gemm_dev": (C.c_int, [_vp, C.c_int, C.c_int, _vp, C.c_int, C.c_int, _vp,
                                              C.c_int, _vp, _vp]),
        "gq_hip_prefill_gate_up_dev": (C.c_int, [_vp, C.c_int, _vp, _vp, C.c_int, C.c_int, _vp, C.c_int,
                                                 _vp]),
        "gq_hip_prefill_attention_dev": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp,
                                                   _vp, _vp]),
        "gq_hip_chat_turn": (C.c_int, [_vp, C.POINTER(C.c_int32), C.c_int, C.POINTER(C.c_int), C.c_int, C.c_int,
                                          C.c_float, C.c_int, C.c_float, C.POINTER(C.c_int), C.POINTER(C.c_int32)]),
        "gq_hip_prefill": (C.c_int, [_vp, C.POINTER(C.c_int32), C.c_int, C.c_int, _fp, _fp,
                                     C.POINTER(C.c_float)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    return L, tuple(sig)


lib, EXPORTS = _load()
NCLASS = 7
CLASS_NAMES = ("qkv", "attention", "o_proj", "gate_up", "down", "lm_head", "other")
MATVEC_PATHS = ("valu", "auto", "mfma", "auto_q6k_ref")


class matvec_path:
    """Context manager selecting the matvec kernels: "auto" (default) the
    int8 matrix-core kernel for gate/up and the LM head of a bound model and
    the vector-ALU kernel for the rest; "valu" the vector-ALU kernel for
    every launch; "mfma" the int8 matrix-core kernel wherever it fits
    (Q4_K/Q6_K; the op-level entry points tile their weights per call),
    else the vector-ALU kernel; "auto_q6k_ref" as "auto" with the Q6_K down
    projection read from the reference layout instead of the unit-layout
    copy made at model bind."""

    def __init__(self, name):
        self.lds = MATVEC_PATHS.index(name)

    def __enter__(self):
        self.prev = lib.gq_hip_set_matvec_path(self.lds)
        return self

    def __exit__(self, *exc):
        lib.gq_hip_set_matvec_path(self.prev)


class GqWeight(C.Structure):
    _fields_ = [("data", _vp), ("dtype", C.c_int), ("rows", C.c_int), ("cols", C.c_int)]


class GqLayer(C.Structure):
    _fields_ = [(n, GqWeight) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")] + [
        ("rms_att", _vp), ("rms_ffn", _vp)]


class GqModel(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "hidden", "ff", "n_heads", "n_kv_heads",
                                      "head_dim", "vocab")] + [
        ("rope_theta", C.c_float), ("rms_eps", C.c_float), ("layers", C.POINTER(GqLayer)),
        ("embed", GqWeight), ("lm_head", GqWeight), ("rms_final", _vp)]


def mem_info(device_id=0):
    """(free, total) bytes of the device (hipMemGetInfo)."""
    f, t = C.c_size_t(0), C.c_size_t(0)
    if lib.gq_hip_mem_info(device_id, C.byref(f), C.byref(t)) != 0:
        raise HipError(f"mem_info({device_id}) failed")
    return f.value, t.value


def device_count() -> int:
    return int(lib.gq_hip_device_count())


def _f(a):
    return a.ctypes.data_as(_fp)


class DevBuf:
    """A device allocation owned by a Context."""

    def __init__(self, ctx, nbytes):
        self.ctx, self.nbytes = ctx, int(nbytes)
        self.ptr = lib.gq_hip_malloc(ctx.h, self.nbytes)
        if not self.ptr:
            ctx.raise_last("gq_hip_malloc")

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        self.ctx.check(lib.gq_hip_h2d(self.ctx.h, self.ptr, arr.ctypes.data, arr.nbytes), "h2d")
        return self

    def download(self, dtype=np.float32, count=None):
        dt = np.dtype(dtype)
        n = self.nbytes // dt.itemsize if count is None else count
        out = np.empty(n, dt)
        self.ctx.check(lib.gq_hip_d2h(self.ctx.h, out.ctypes.data, self.ptr, out.nbytes), "d2h")
        return out

    def free(self):
        if self.ptr:
            lib.gq_hip_free(self.ctx.h, self.ptr)
            self.ptr = None


class Context:
    """One device context: stream, allocations, KV cache, bound model."""

    def __init__(self, device_id=0):
        self.h = lib.gq_hip_create(device_id)
        if not self.h:
            raise HipError(f"no usable HIP device {device_id} (device_count={device_count()})")
        self._keep = []

    def close(self):
        if self.h:
            lib.gq_hip_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def raise_last(self, what, rc=None):
        msg = lib.gq_hip_last_error(self.h).decode(errors="replace")
        raise HipError(f"{what} failed (rc={rc}): {msg}")

    def check(self, rc, what):
        if rc != 0:
            self.raise_last(what, rc)
        return rc

    def info(self):
        n = C.c_int()
        name = C.create_string_buffer(128)
        lib.gq_hip_device_info(self.h, C.byref(n), name, 128)
        return n.value, name.value.decode()

    def sync(self):
        self.check(lib.gq_hip_sync(self.h), "sync")

    # ---- memory ----
    def alloc(self, nbytes):
        return DevBuf(self, nbytes)

    def upload(self, arr):
        return DevBuf(self, np.asarray(arr).nbytes).upload(arr)

    def upload_weight(self, arr):
        arr = np.ascontiguousarray(arr)
        p = lib.gq_hip_upload_weight(self.h, arr.ctypes.data, arr.nbytes)
        if not p:
            self.raise_last("upload_weight")
        return p

    # ---- synthetic inputs ----
    def synth_quant(self, dtype, rows, cols, seed):
        """Blocks of a generator code: a dtype, or Q4_K | SYNTH_Q4K_ZERO_MEAN."""
        buf = DevBuf(self, S.qbytes(dtype & ~S.SYNTH_Q4K_ZERO_MEAN, rows, cols))
        self.check(lib.gq_hip_synth_quant(self.h, buf.ptr, dtype, rows, cols, seed), "synth_quant")
        return buf

    def synth_normal(self, n, seed):
        buf = DevBuf(self, 4 * n)
        self.check(lib.gq_hip_synth_normal(self.h, buf.ptr, n, seed), "synth_normal")
        return buf

    def synth_norm_weight(self, n, seed, shift=0):
        """(1 + N(0,1)/64) * 2^-shift; the power-of-two scale is applied on
        the host (exact), like the oracle's."""
        buf = DevBuf(self, 4 * n)
        self.check(lib.gq_hip_synth_norm_weight(self.h, buf.ptr, n, seed), "synth_norm_weight")
        if shift:
            buf.upload(np.ldexp(buf.download(count=n), -shift).astype(np.float32))
        return buf

    # ---- ops ----
    def matvec_host(self, dtype, w_ptr, rows, cols, x, byte_size=0):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(rows, np.float32)
        rc = lib.gq_hip_matvec(self.h, dtype, w_ptr, rows, cols, byte_size, _f(x), _f(y))
        return rc, y

    def matvec_dev(self, dtype, w_ptr, rows, cols, x_buf, y_buf):
        self.check(lib.gq_hip_matvec_dev(self.h, dtype, w_ptr, rows, cols, x_buf.ptr, y_buf.ptr),
                   "matvec_dev")

    def matvec_norm_dev(self, dtype, w_ptr, rows, cols, x_buf, nw_buf, eps, y_buf):
        self.check(lib.gq_hip_matvec_norm_dev(self.h, dtype, w_ptr, rows, cols, x_buf.ptr, nw_buf.ptr,
                                              eps, y_buf.ptr), "matvec_norm_dev")

    def rmsnorm_dev(self, x_buf, w_buf, out_buf, dim, eps):
        self.check(lib.gq_hip_rmsnorm_dev(self.h, x_buf.ptr, w_buf.ptr if w_buf else None,
                                          out_buf.ptr, dim, eps), "rmsnorm")

    def silu_mul_dev(self, g_buf, u_buf, n):
        self.check(lib.gq_hip_silu_mul_dev(self.h, g_buf.ptr, u_buf.ptr, n), "silu_mul")

    def embed_dev(self, dtype, table_ptr, hidden, token, out_buf):
        self.check(lib.gq_hip_embed_dev(self.h, dtype, table_ptr, hidden, token, out_buf.ptr),
                   "embed")

    def argmax_dev(self, x_buf, n):
        out = DevBuf(self, 4)
        self.check(lib.gq_hip_argmax_dev(self.h, x_buf.ptr, n, out.ptr), "argmax")
        v = int(out.download(np.int32)[0])
        out.free()
        return v

    # ---- KV cache ----
    def kv_init(self, n_layers, n_kv_heads, head_dim, max_seq, rope_theta):
        self.kv_geom = (n_layers, n_kv_heads, head_dim, max_seq)
        self.check(lib.gq_hip_kv_init(self.h, n_layers, n_kv_heads, head_dim, max_seq, rope_theta),
                   "kv_init")

    def kv_layer_floats(self):
        _, nkv, hd, ms = self.kv_geom
        return nkv * ms * hd

    def kv_append(self, layer, pos, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        return lib.gq_hip_kv_append(self.h, layer, pos, _f(k), _f(v))

    def kv_read_layer(self, layer):
        n = self.kv_layer_floats()
        k = np.empty(n, np.float32)
        v = np.empty(n, np.float32)
        self.check(lib.gq_hip_kv_read_layer(self.h, layer, _f(k), _f(v)), "kv_read_layer")
        return k, v

    def kv_write_layer(self, layer, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self.check(lib.gq_hip_kv_write_layer(self.h, layer, _f(k), _f(v)), "kv_write_layer")

    def kv_sync(self, layer, pos, T, hk, hv, head_stride, max_seq):
        return lib.gq_hip_kv_sync(self.h, layer, pos, T, _f(hk), _f(hv), head_stride, max_seq)

    def kv_prefill_synth(self, seed_k, seed_v, n_pos):
        self.check(lib.gq_hip_kv_prefill_synth(self.h, seed_k, seed_v, n_pos), "kv_prefill")

    def rope_append_dev(self, layer, pos, n_heads, q_buf, k_buf, v_buf):
        return lib.gq_hip_rope_append_dev(self.h, layer, pos, n_heads, q_buf.ptr, k_buf.ptr,
                                          v_buf.ptr)

    def attention_dev(self, layer, pos, n_heads, q_buf, out_buf):
        return lib.gq_hip_attention_dev(self.h, layer, pos, n_heads, q_buf.ptr, out_buf.ptr)

    def attention_dev_noalloc(self, layer, pos, n_heads, q_buf, out_buf):
        """gq_hip_attention_dev with the partials in the library's static
        device scratch: no allocation, calls on one GPU must not overlap."""
        return lib.gq_hip_attention_dev_noalloc(self.h, layer, pos, n_heads, q_buf.ptr, out_buf.ptr)

    def prefill_attention_dev(self, layer, pos, T, n_heads, q_buf, k_buf, v_buf, out_buf):
        return lib.gq_hip_prefill_attention_dev(self.h, layer, pos, T, n_heads, q_buf.ptr, k_buf.ptr,
                                                v_buf.ptr, out_buf.ptr)

    # ---- sessions ----
    def lctx_save(self, path, current_pos, tokens=None):
        toks = np.ascontiguousarray(tokens if tokens is not None else [], np.int32)
        return lib.gq_hip_lctx_save(self.h, path.encode(), current_pos,
                                    toks.ctypes.data_as(C.POINTER(C.c_int32)), toks.size)

    def lctx_load(self, path):
        pos = C.c_int(-1)
        n = C.c_int(0)
        toks = C.POINTER(C.c_int32)()
        rc = lib.gq_hip_lctx_load(self.h, path.encode(), C.byref(pos), C.byref(toks), C.byref(n))
        if rc:
            return rc, None, None
        t = np.ctypeslib.as_array(toks, shape=(n.value,)).copy() if n.value > 0 else np.zeros(0, np.int32)
        if n.value > 0:
            C.CDLL(None).free(toks)
        return 0, pos.value, t

    def prompt_cache_save(self, path, prefix_len):
        return lib.gq_hip_prompt_cache_save(self.h, prefix_len, path.encode())

    def prompt_cache_load(self, path):
        n = C.c_int(-1)
        rc = lib.gq_hip_prompt_cache_load(self.h, path.encode(), C.byref(n))
        return rc, n.value

    def lctx_restore_image(self, image_ptr, size):
        pos = C.c_int(-1)
        ms = C.c_float(0)
        rc = lib.gq_hip_lctx_restore_image(self.h, image_ptr, size, C.byref(pos), C.byref(ms))
        return rc, pos.value, ms.value


class DeviceModel:
    """A synthetic model (guanaco_amd.spec) generated directly in HBM and bound
    to a Context, with its KV cache pre-filled."""

    def __init__(self, ctx: Context, spec: S.ModelSpec, max_seq: int, prefill: int = 0):
        self.ctx, self.spec, self.max_seq = ctx, spec, max_seq
        s = spec
        from .synth import tensor_seed  # pure function of the seed
        ctx.kv_init(s.n_layers, s.n_kv_heads, s.head_dim, max_seq, s.rope_theta)
        self.bufs = []
        layers = (GqLayer * s.n_layers)()
        names = dict(wq="wq", wk="wk", wv="wv", wo="wo", wg="w_gate", wu="w_up", wd="w_down")
        for l in range(s.n_layers):
            dts = s.dtypes(l)
            for k, field in names.items():
                rows, cols = s.shape(k)
                b = ctx.synth_quant(s.gen(dts[k]), rows, cols, tensor_seed(s.seed, l, S.SLOT[k]))
                self.bufs.append(b)
                setattr(layers[l], field, GqWeight(b.ptr, dts[k], rows, cols))
            ra = ctx.synth_norm_weight(s.hidden, tensor_seed(s.seed, l, S.SLOT["rms_att"]), s.norm_shift)
            rf = ctx.synth_norm_weight(s.hidden, tensor_seed(s.seed, l, S.SLOT["rms_ffn"]), s.norm_shift)
            self.bufs += [ra, rf]
            layers[l].rms_att, layers[l].rms_ffn = ra.ptr, rf.ptr
        emb = ctx.synth_quant(s.gen(s.embed_dtype), s.vocab, s.hidden, tensor_seed(s.seed, -1, S.SLOT["embed"]))
        lm = ctx.synth_quant(s.gen(s.lm_head_dtype), s.vocab, s.hidden,
                             tensor_seed(s.seed, -1, S.SLOT["lm_head"]))
        rfin = ctx.synth_norm_weight(s.hidden, tensor_seed(s.seed, -1, S.SLOT["rms_final"]), s.norm_shift)
        self.bufs += [emb, lm, rfin]
        self.layers = layers
        self.model = GqModel(s.n_layers, s.hidden, s.ff, s.n_heads, s.n_kv_heads, s.head_dim, s.vocab,
                             s.rope_theta, s.rms_eps, C.cast(layers, C.POINTER(GqLayer)),
                             GqWeight(emb.ptr, s.embed_dtype, s.vocab, s.hidden),
                             GqWeight(lm.ptr, s.lm_head_dtype, s.vocab, s.hidden), rfin.ptr)
        ctx.check(lib.gq_hip_model_bind(ctx.h, C.byref(self.model)), "model_bind")
        if prefill:
            ctx.kv_prefill_synth(tensor_seed(s.seed, -1, S.SLOT["kv_k"]),
                                 tensor_seed(s.seed, -1, S.SLOT["kv_v"]), prefill)

    def weight(self, layer, slot):
        names = dict(wq="wq", wk="wk", wv="wv", wo="wo", wg="w_gate", wu="w_up", wd="w_down")
        return getattr(self.layers[layer], names[slot])

    def forward(self, token, pos, want_logits=True, want_hidden=False):
        s = self.spec
        logits = np.empty(s.vocab, np.float32) if want_logits else None
        hid = np.empty(s.n_layers * s.hidden, np.float32) if want_hidden else None
        tok = lib.gq_hip_forward_token(self.ctx.h, token, pos, _f(logits) if want_logits else None,
                                       _f(hid) if want_hidden else None)
        if tok < 0:
            self.ctx.raise_last("forward_token", tok)
        return tok, logits, (hid.reshape(s.n_layers, s.hidden) if want_hidden else None)

    def prefill(self, tokens, pos, want_logits=True, want_hidden=False):
        """forward() over a prompt: returns (next greedy token, logits of the
        last token, its hidden state before the final norm, device ms)."""
        s = self.spec
        toks = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(s.vocab, np.float32) if want_logits else None
        hid = np.empty(s.hidden, np.float32) if want_hidden else None
        ms = C.c_float(0)
        tok = lib.gq_hip_prefill(self.ctx.h, toks.ctypes.data_as(C.POINTER(C.c_int32)), toks.size, pos,
                                 _f(logits) if want_logits else None, _f(hid) if want_hidden else None,
                                 C.byref(ms))
        if tok < 0:
            self.ctx.raise_last("prefill", tok)
        return tok, logits, hid, ms.value

    def chat_turn(self, tokens, current_pos, max_tokens, eos_token, temperature=0.0, top_k=40, top_p=0.9,
                  rnd=None):
        """gq_hip_chat_turn: (status, reply tokens, new current_pos); status
        -6 when the turn does not fit (restart the conversation)."""
        toks = np.ascontiguousarray(tokens, np.int32)
        pos = C.c_int(current_pos)
        reply = np.zeros(max(1, max_tokens), np.int32)
        r = None if rnd is None else np.ascontiguousarray(rnd, np.int32)
        n = lib.gq_hip_chat_turn(self.ctx.h, toks.ctypes.data_as(C.POINTER(C.c_int32)), toks.size, C.byref(pos),
                                 max_tokens, eos_token, temperature, top_k, top_p,
                                 r.ctypes.data_as(C.POINTER(C.c_int)) if r is not None else None,
                                 reply.ctypes.data_as(C.POINTER(C.c_int32)))
        if n < 0:
            return n, None, current_pos
        return 0, reply[:n].copy(), pos.value

    def decode_loop(self, token, pos, n_steps, use_graph=True):
        out = np.zeros(n_steps, np.int32)
        ms = C.c_float(0)
        self.ctx.check(lib.gq_hip_decode_loop(self.ctx.h, token, pos, n_steps, 1 if use_graph else 0,
                                              out.ctypes.data_as(C.POINTER(C.c_int32)), C.byref(ms)),
                       "decode_loop")
        return out, ms.value

    def time_op(self, op, pos, n_iter=64):
        """Average ms of one op (a CLASS_NAMES entry other than "other")
        launched n_iter times back to back over the layers."""
        ms = lib.gq_hip_time_op(self.ctx.h, CLASS_NAMES.index(op), pos, n_iter)
        if ms < 0:
            self.ctx.raise_last("time_op")
        return float(ms)

    def profile_step(self, token, pos):
        ms = (C.c_double * NCLASS)()
        n = (C.c_int * NCLASS)()
        b = (C.c_double * NCLASS)()
        self.ctx.check(lib.gq_hip_profile_step(self.ctx.h, token, pos, ms, n, b), "profile_step")
        return {CLASS_NAMES[i]: dict(ms=ms[i], launches=n[i], bytes=b[i]) for i in range(NCLASS)}

    def transformer_layer(self, layer, pos, hidden, hk=None, hv=None, head_stride=0):
        hidden = np.ascontiguousarray(hidden, np.float32)
        rc = lib.gq_hip_transformer_layer(self.ctx.h, layer, pos, _f(hidden),
                                          _f(hk) if hk is not None else None,
                                          _f(hv) if hv is not None else None, head_stride)
        return rc, hidden
