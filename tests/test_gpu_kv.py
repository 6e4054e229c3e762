"""Device KV cache: append / gather / sync, fused RoPE+append and .lctx
sessions are bit-exact against the oracle (pinned to the reference's
kv_cache.c and session.c in test_oracle.py)."""
import ctypes as C

import numpy as np
import pytest

from oracle import HostKV, fptr, u8ptr
from guanaco_amd import spec as S
from util import bits

pytestmark = pytest.mark.gpu

GEOM = (2, 2, 8, 16)  # layers, kv heads, head_dim, max_seq


def fresh(ctx, geom=GEOM, theta=500000.0):
    ctx.kv_init(*geom, theta)
    return HostKV(*geom)


def test_append_gather_bitexact_with_wrap(ctx, orc):
    kv = fresh(ctx)
    rng = np.random.default_rng(1)
    for layer, pos in ((0, 0), (1, 5), (1, 15), (0, 16 + 3), (1, 5)):
        k = rng.standard_normal(16).astype(np.float32)
        v = rng.standard_normal(16).astype(np.float32)
        assert ctx.kv_append(layer, pos, k, v) == 0
        assert orc.lib.orc_kv_append(C.byref(kv.s), layer, pos, fptr(k), fptr(v)) == 0
    for layer in range(2):
        dk, dv = ctx.kv_read_layer(layer)
        n = kv.k.size // 2
        assert np.array_equal(bits(dk), bits(kv.k[layer * n:(layer + 1) * n]))
        assert np.array_equal(bits(dv), bits(kv.v[layer * n:(layer + 1) * n]))


def test_append_rejects_bad_input(ctx):
    fresh(ctx)
    k = np.zeros(16, np.float32)
    assert ctx.kv_append(0, -1, k, k) == -5
    assert ctx.kv_append(2, 0, k, k) == -1
    assert ctx.kv_append(-1, 0, k, k) == -1


def test_sync_rows(ctx):
    """cuda_sync_kv_cache semantics: T host rows from pos -> device."""
    fresh(ctx)
    L, nkv, hd, ms = GEOM
    hk = np.random.default_rng(2).standard_normal(nkv * ms * hd).astype(np.float32)
    hv = -hk
    assert ctx.kv_sync(1, 4, 3, hk, hv, ms * hd, ms) == 0
    dk, dv = ctx.kv_read_layer(1)
    dk = dk.reshape(nkv, ms, hd)
    exp = hk.reshape(nkv, ms, hd)
    assert np.array_equal(dk[:, 4:7], exp[:, 4:7]) and not dk[:, :4].any() and not dk[:, 7:].any()
    assert ctx.kv_sync(1, 14, 3, hk, hv, ms * hd, ms) == -5
    assert ctx.kv_sync(1, 0, 1, hk, hv, ms * hd, ms + 1) == -1


def test_lctx_save_bytes_and_restore(ctx, orc, tmp_path):
    kv = fresh(ctx)
    kv.prefill(orc, S.TINY_TEST, 11)
    for l in range(2):
        n = kv.k.size // 2
        ctx.kv_write_layer(l, kv.k[l * n:(l + 1) * n], kv.v[l * n:(l + 1) * n])
    toks = np.array([9, 8, 7, 6, 5], np.int32)
    path = str(tmp_path / "a.lctx")
    assert ctx.lctx_save(path, 11, toks) == 0
    size = orc.lib.orc_lctx_size(C.byref(kv.s), 5)
    img = np.zeros(size, np.uint8)
    orc.lib.orc_lctx_write(C.byref(kv.s), 11, toks.ctypes.data_as(C.POINTER(C.c_int32)), 5,
                           u8ptr(img), size)
    assert np.array_equal(np.fromfile(path, np.uint8), img)
    # wipe and restore from the file
    fresh(ctx)
    rc, pos, t = ctx.lctx_load(path)
    assert rc == 0 and pos == 11 and np.array_equal(t, toks)
    for l in range(2):
        n = kv.k.size // 2
        dk, dv = ctx.kv_read_layer(l)
        assert np.array_equal(bits(dk), bits(kv.k[l * n:(l + 1) * n]))
        assert np.array_equal(bits(dv), bits(kv.v[l * n:(l + 1) * n]))
    # restore from an in-memory image
    fresh(ctx)
    rc, pos, ms = ctx.lctx_restore_image(img.ctypes.data, img.nbytes)
    assert rc == 0 and pos == 11 and ms >= 0
    dk, _ = ctx.kv_read_layer(1)
    assert np.array_equal(bits(dk), bits(kv.k[kv.k.size // 2:]))


def test_lctx_rejects_mismatch(ctx, tmp_path):
    fresh(ctx)
    path = str(tmp_path / "b.lctx")
    assert ctx.lctx_save(path, 3) == 0
    fresh(ctx, (2, 2, 8, 32))  # different max_seq (session.c:141-145)
    assert ctx.lctx_load(path)[0] == -1
    fresh(ctx, (3, 2, 8, 16))  # different layer count (session.c:132-139)
    assert ctx.lctx_load(path)[0] == -1
    raw = bytearray(open(path, "rb").read())
    raw[0] ^= 1  # bad magic
    open(path, "wb").write(bytes(raw))
    fresh(ctx)
    assert ctx.lctx_load(path)[0] == -1


@pytest.mark.parametrize("nh,nkv,hd,pos,theta", [
    (8, 2, 64, 5, 500000.0), (32, 8, 128, 8191, 500000.0), (32, 4, 64, 639, 500000.0),
    # TinyLlama's rope theta (config 2) at its shape, and at the 8B shape
    (32, 4, 64, 639, 10000.0), (32, 4, 64, 2047, 10000.0), (32, 8, 128, 4095, 10000.0),
])
@pytest.mark.parametrize("off", [0, 1])
def test_rope_append_bitexact(ctx, orc, nh, nkv, hd, pos, theta, off):
    """Fused RoPE + append: rotated q and the cached K row equal the
    reference's rope() + kv_cache_append bit for bit (table from the same fp32
    expressions, no contraction).  off = 1 passes q, k and v one float past
    an 8-byte boundary: the kernel's scalar path for such buffers."""
    ms = pos + 1
    ctx.kv_init(1, nkv, hd, ms, theta)
    rng = np.random.default_rng(pos)
    q = rng.standard_normal(nh * hd).astype(np.float32) * np.float32(30)
    k = rng.standard_normal(nkv * hd).astype(np.float32) * np.float32(30)
    v = rng.standard_normal(nkv * hd).astype(np.float32)
    pad = np.zeros(off, np.float32)
    qb, kb, vb = (ctx.upload(np.concatenate([pad, a])) for a in (q, k, v))
    at = [type("At", (), {"ptr": b.ptr + 4 * off})() for b in (qb, kb, vb)]
    assert ctx.rope_append_dev(0, pos, nh, *at) == 0
    q2, k2 = orc.rope(q, k, nh, nkv, hd, pos, theta)
    assert np.array_equal(bits(qb.download()[off:]), bits(q2))
    dk, dv = ctx.kv_read_layer(0)
    dk = dk.reshape(nkv, ms, hd)
    dv = dv.reshape(nkv, ms, hd)
    assert np.array_equal(bits(dk[:, pos]), bits(k2.reshape(nkv, hd)))
    assert np.array_equal(bits(dv[:, pos]), bits(v.reshape(nkv, hd)))
    assert ctx.rope_append_dev(0, ms, nh, *at) == -5
