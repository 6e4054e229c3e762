"""The weight upload path (cuda_upload_weight's replacement,
matvec_q4k_cuda.cu:115-133; the loader's call, loader.c:701-728):

* from a real private file mapping (mmap MAP_PRIVATE, as the reference's
  GGUF loader maps the model), sizes that do and do not fill the 32 MiB
  staging chunks, bytes on the device equal to the file's;
* gq_hip_destroy returns every byte: hipMemGetInfo's free memory after a
  context that uploaded weights, built a KV cache and bound a model is what
  it was before the context (after one warm-up context, which loads the
  code objects)."""
import ctypes as C
import mmap
import os

import numpy as np
import pytest

import guanaco_amd.hip as H
from guanaco_amd import spec as S

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("size", [(1 << 20) + 17, (96 << 20) + 12345, 64 << 20])
def test_upload_from_private_file_mapping(ctx, tmp_path, size):
    path = tmp_path / "w.bin"
    data = np.random.default_rng(size).integers(0, 256, size, dtype=np.uint8)
    data.tofile(path)
    with open(path, "rb") as f:
        mm = mmap.mmap(f.fileno(), 0, flags=mmap.MAP_PRIVATE, prot=mmap.PROT_READ | mmap.PROT_WRITE)
    try:
        addr = C.addressof(C.c_char.from_buffer(mm))
        d = H.lib.gq_hip_upload_weight(ctx.h, addr, size)
        assert d, H.lib.gq_hip_last_error(ctx.h)
        back = np.empty(size, np.uint8)
        ctx.check(H.lib.gq_hip_d2h(ctx.h, back.ctypes.data, d, size), "d2h")
        assert np.array_equal(back, data)
        H.lib.gq_hip_free(ctx.h, d)
    finally:
        del addr
        mm.close()


def test_destroy_returns_every_byte(orc):
    def cycle():
        c = H.Context(0)
        dm = H.DeviceModel(c, S.TINY_TEST, 256, prefill=16)
        w = np.random.default_rng(1).integers(0, 256, 200 << 20, dtype=np.uint8)
        p = H.lib.gq_hip_upload_weight(c.h, w.ctypes.data, w.nbytes)
        assert p and dm.forward(3, 16)[0] >= 0
        c.sync()
        c.close()

    cycle()  # warm-up: code objects, the static scratch array, runtime pools
    free0, total = H.mem_info(0)
    cycle()
    free1, _ = H.mem_info(0)
    print(f"free before {free0 / 2**30:.3f} GiB, after {free1 / 2**30:.3f} GiB of {total / 2**30:.1f}")
    assert free1 == free0, f"{(free0 - free1) / 2**20:.2f} MiB not returned"
