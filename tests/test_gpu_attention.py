"""Split-K GQA decode attention against the oracle's restatement of the
reference (engine.c:433-509) on seeded N(0,1) K/V and N(0,1) queries (the
config-4 setting), at the 8B shape up to 32768 positions (64- and
128-position chunks), the TinyLlama shape and edge lengths.  Tolerance:
relative L2 <= 1e-5."""
import numpy as np
import pytest

from oracle import HostKV
from guanaco_amd import spec as S
from util import rel_l2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nh,nkv,hd,L,ms", [
    (32, 8, 128, 8192, 8320),   # 8B shape at ctx 8192
    (32, 8, 128, 513, 8320),
    (32, 8, 128, 1, 8320),      # a single position
    (32, 4, 64, 513, 640),      # TinyLlama shape
    (32, 4, 64, 640, 640),      # cache exactly full
    (8, 8, 64, 77, 96),         # no grouping (G = 1)
    (64, 8, 128, 1000, 1024),   # G = 8 at head_dim 128
    (32, 8, 128, 12289, 12400),  # 128-position chunks (caches past 12288)
    (32, 8, 128, 16384, 16384),  # config 4 at ctx 16384, cache exactly full
    (32, 8, 128, 32768, 32768),  # config 4 at ctx 32768: 256 chunks of 128 in the merge
    (32, 4, 64, 13000, 13000),   # 128-position chunks at head_dim 64
])
def test_attention_vs_oracle(ctx, orc, nh, nkv, hd, L, ms):
    ctx.kv_init(1, nkv, hd, ms, 500000.0)
    seed_k = 0xA11CE + L
    seed_v = 0xB0B + L
    ctx.kv_prefill_synth(seed_k, seed_v, L)
    kv = HostKV(1, nkv, hd, ms)
    from oracle import fptr
    for arr, seed in ((kv.k, seed_k), (kv.v, seed_v)):
        orc.lib.orc_synth_kv(seed, fptr(arr), 1, nkv, hd, ms, L)
    dk, dv = ctx.kv_read_layer(0)
    assert np.array_equal(dk, kv.k) and np.array_equal(dv, kv.v)
    q = orc.synth_normal(7 * L + nh, nh * hd)
    qb, ob = ctx.upload(q), ctx.alloc(4 * nh * hd)
    assert ctx.attention_dev(0, L - 1, nh, qb, ob) == 0
    ref = orc.attention(q, kv, 0, nh, L - 1)
    assert rel_l2(ob.download(), ref) < 1e-5


def test_attention_rejects_bad_position(ctx):
    ctx.kv_init(1, 2, 64, 32, 500000.0)
    qb, ob = ctx.alloc(4 * 8 * 64), ctx.alloc(4 * 8 * 64)
    assert ctx.attention_dev(0, 32, 8, qb, ob) == -5
    assert ctx.attention_dev(0, -1, 8, qb, ob) == -5
    assert ctx.attention_dev(0, 3, 7, qb, ob) == -1
