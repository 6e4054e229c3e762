"""Session files at full size and the frozen-prefix prompt cache, on the
device cache:

* the config-4 restore: a 4096-token prefix of the 8B shape (32 layers x 8
  KV heads x 128 x max_seq 4096, 1 GiB of K/V) saved from the device, read
  into pinned host memory and restored with gq_hip_lctx_restore_image; every
  layer's K and V is bit-exact against the oracle's synthesis of the same
  seeds (session.c:107-188);
* prompt_cache_save / prompt_cache_load (session.c:192-251): the device file
  is byte-identical to the oracle's image with current_pos = prefix_len and
  no tokens (pinned to the reference's prompt_cache_save in test_oracle.py),
  and loads back bit-exact."""
import ctypes as C
import os

import numpy as np
import pytest

import guanaco_amd.hip as H
from oracle import HostKV, fptr, u8ptr
from guanaco_amd import spec as S
from util import bits

pytestmark = pytest.mark.gpu


def test_prompt_cache_bytes_and_load(ctx, orc, tmp_path):
    geom = (2, 2, 8, 32)
    ctx.kv_init(*geom, 500000.0)
    kv = HostKV(*geom)
    kv.prefill(orc, S.TINY_TEST, 13)
    n = kv.k.size // 2
    for l in range(2):
        ctx.kv_write_layer(l, kv.k[l * n:(l + 1) * n], kv.v[l * n:(l + 1) * n])
    path = str(tmp_path / "p.lctx")
    assert ctx.prompt_cache_save(path, 0) == -1  # prefix_len <= 0 (session.c:194)
    assert ctx.prompt_cache_save(path, 13) == 0
    size = orc.lib.orc_lctx_size(C.byref(kv.s), 0)
    img = np.zeros(size, np.uint8)
    orc.lib.orc_lctx_write(C.byref(kv.s), 13, None, 0, u8ptr(img), size)
    assert np.array_equal(np.fromfile(path, np.uint8), img)
    ctx.kv_init(*geom, 500000.0)  # a fresh, zeroed cache
    rc, prefix = ctx.prompt_cache_load(path)
    assert rc == 0 and prefix == 13
    for l in range(2):
        dk, dv = ctx.kv_read_layer(l)
        assert np.array_equal(bits(dk), bits(kv.k[l * n:(l + 1) * n]))
        assert np.array_equal(bits(dv), bits(kv.v[l * n:(l + 1) * n]))
    # a session file with a token history loads as a prompt cache as well
    # (prompt_cache_load is kv_cache_load without the tokens)
    path2 = str(tmp_path / "s.lctx")
    assert ctx.lctx_save(path2, 9, np.array([4, 5, 6], np.int32)) == 0
    assert ctx.prompt_cache_load(path2) == (0, 9)


def test_lctx_restore_4096_prefix_1gib_pinned(ctx, orc, tmp_path):
    L, nkv, hd, ms = 32, 8, 128, 4096
    sk, sv = 0x5EED1, 0x5EED2
    print(f"lctx restore: {L} layers x {nkv} x {hd} x {ms}", flush=True)
    ctx.kv_init(L, nkv, hd, ms, 500000.0)
    ctx.kv_prefill_synth(sk, sv, ms)
    toks = (np.arange(ms, dtype=np.int64) * 7919 % 128256).astype(np.int32)
    path = str(tmp_path / "big.lctx")
    assert ctx.lctx_save(path, ms, toks) == 0
    kv_bytes = 2 * L * nkv * ms * hd * 4
    size = os.path.getsize(path)
    assert size == 64 + 4 * ms + kv_bytes
    img = H.lib.gq_hip_host_alloc_pinned(size)
    assert img, "pinned allocation failed"
    try:
        with open(path, "rb") as f:
            assert f.readinto((C.c_char * size).from_address(img)) == size
        os.unlink(path)
        hdr = np.frombuffer((C.c_char * 64).from_address(img), np.int32)
        assert list(hdr[1:8]) == [1, L, nkv, hd, ms, ms, ms]
        ctx.kv_prefill_synth(99, 98, ms)  # overwrite the cache before restoring
        rc, pos, t_ms = ctx.lctx_restore_image(img, size)
        assert rc == 0 and pos == ms
        print(f"restored {kv_bytes / 2**30:.2f} GiB in {t_ms:.1f} ms "
              f"({kv_bytes / t_ms / 1e6:.1f} GB/s)", flush=True)
    finally:
        H.lib.gq_hip_host_free_pinned(img)
    hk = HostKV(L, nkv, hd, ms)
    orc.lib.orc_synth_kv(sk, fptr(hk.k), L, nkv, hd, ms, ms)
    orc.lib.orc_synth_kv(sv, fptr(hk.v), L, nkv, hd, ms, ms)
    n = nkv * ms * hd
    for l in range(L):
        dk, dv = ctx.kv_read_layer(l)
        assert np.array_equal(bits(dk), bits(hk.k[l * n:(l + 1) * n])), f"K layer {l}"
        assert np.array_equal(bits(dv), bits(hk.v[l * n:(l + 1) * n])), f"V layer {l}"
