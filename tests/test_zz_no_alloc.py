"""gq_hip_attention_dev_noalloc (split-K partials in the library's static
device scratch, no allocation) against gq_hip_attention_dev (partials in
allocated memory): the same kernels on the same inputs, so the outputs must
be bit-identical, on two calls in a row, the second over fewer positions, in
a context with no bound model (where gq_hip_attention_dev allocates) and in
one whose partials would not fit the scratch (a clear error, no launch)."""
import numpy as np
import pytest

import guanaco_amd.hip as H

pytestmark = pytest.mark.gpu


def _bits(buf, n):
    return buf.download(np.float32, n).view(np.uint32)


def test_noalloc_attention_matches_allocating_entry_point():
    n_kv, hd, nh, ms = 8, 128, 32, 4096
    with H.Context(0) as ctx:
        ctx.kv_init(2, n_kv, hd, ms, 500000.0)
        ctx.kv_prefill_synth(11, 12, ms)
        q = ctx.synth_normal(nh * hd, 13)
        oa, ob = ctx.alloc(4 * nh * hd), ctx.alloc(4 * nh * hd)
        for layer, pos in ((1, ms - 1), (0, 700)):
            print(f"noalloc attention layer {layer} pos {pos}", flush=True)
            assert ctx.attention_dev(layer, pos, nh, q, oa) == 0
            assert ctx.attention_dev_noalloc(layer, pos, nh, q, ob) == 0, H.lib.gq_hip_last_error(ctx.h)
            ctx.sync()
            a, b = _bits(oa, nh * hd), _bits(ob, nh * hd)
            assert np.isfinite(a.view(np.float32)).all()
            assert np.array_equal(a, b), f"layer {layer} pos {pos}: {np.count_nonzero(a != b)} words differ"


def test_noalloc_attention_rejects_partials_beyond_scratch():
    # 32 heads x 1024 chunks x 130 floats = 4.26M floats > the 2M-float scratch
    with H.Context(0) as ctx:
        ctx.kv_init(1, 1, 128, 131072, 500000.0)
        q, o = ctx.alloc(4 * 32 * 128), ctx.alloc(4 * 32 * 128)
        assert ctx.attention_dev_noalloc(0, 5, 32, q, o) == -1
        assert b"scratch" in H.lib.gq_hip_last_error(ctx.h)
