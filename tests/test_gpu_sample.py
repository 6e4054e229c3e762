"""On-device sampling against the reference's own samplers (tokenizer.c:175-333,
compiled from its sources in oracle/_ref/libref.so) on the same libc rand()
stream: for every draw, srand(seed) then the reference's sample_* (which
draws one rand()), and srand(seed) again then rand() for the device.

top-k replays the reference's slot order, top-p sorts stably and plain
temperature sampling sums in the reference's sequential float order, so
every mode must pick the reference's token for every draw, ties included,
except that the device's expf may differ from glibc's in the last bit: a
plain-temperature draw within that of a cumulative boundary may pick the
neighbouring token, and at most one such draw in 64 is allowed there."""
import ctypes as C

import numpy as np
import pytest

from oracle import fptr

pytestmark = pytest.mark.gpu

LIBC = C.CDLL(None)
LIBC.srand.argtypes = [C.c_uint]
LIBC.rand.restype = C.c_int


@pytest.fixture(scope="module")
def samplers(ref):
    L = ref.lib
    L.sample_top_k.argtypes = [C.POINTER(C.c_float), C.c_int, C.c_int, C.c_float]
    L.sample_top_p.argtypes = [C.POINTER(C.c_float), C.c_int, C.c_float, C.c_float]
    L.sample_temperature.argtypes = [C.POINTER(C.c_float), C.c_int, C.c_float]
    for f in (L.sample_top_k, L.sample_top_p, L.sample_temperature):
        f.restype = C.c_int
    return L


def ref_pick(L, logits, temperature, top_k, top_p):
    """generate.c:302-311"""
    V = logits.size
    if temperature <= 0.0:
        return int(L.sample_greedy(fptr(logits), V))
    if 0 < top_k < V:
        return int(L.sample_top_k(fptr(logits), V, top_k, temperature))
    if top_p < 1.0:
        return int(L.sample_top_p(fptr(logits), V, top_p, temperature))
    return int(L.sample_temperature(fptr(logits), V, temperature))


def logits_for(orc, V, kind, seed):
    x = orc.synth_normal(seed, V) * np.float32(3.0)
    if kind == "ties":  # quarter steps: many exactly equal logits
        x = (np.round(x * 4) / 4).astype(np.float32)
    elif kind == "rising":  # larger logits late in the vocabulary (many slot replacements)
        x = (x + np.linspace(0, 12, V, dtype=np.float32)).astype(np.float32)
    return np.ascontiguousarray(x, np.float32)


CASES = [
    # vocab, logits, temperature, top_k, top_p
    (128256, "normal", 0.8, 40, 1.0),
    (128256, "ties", 0.8, 40, 1.0),
    (128256, "rising", 1.0, 40, 1.0),
    (32000, "normal", 1.0, 1, 1.0),
    (32000, "normal", 0.7, 1024, 1.0),
    (32000, "ties", 1.2, 1000, 1.0),
    (128256, "normal", 0.7, 0, 0.9),
    (128256, "ties", 1.0, 0, 0.5),
    (32000, "normal", 1.0, 0, 0.01),
    (32000, "normal", 0.0, 40, 0.9),   # greedy
    (32000, "normal", 1.0, 0, 0.0),    # top_p <= 0: greedy
    (128256, "normal", 1.0, 0, 1.0),   # plain temperature
    (32000, "ties", 0.5, 0, 1.0),
]


@pytest.mark.parametrize("V,kind,T,k,p", CASES)
def test_sample_matches_reference(ctx, orc, samplers, V, kind, T, k, p):
    import guanaco_amd.hip as H
    x = logits_for(orc, V, kind, 17 + V + len(kind))
    xd = ctx.upload(x)
    n, bad = 64, 0
    for d in range(n):
        seed = 1000 + 7 * d
        LIBC.srand(seed)
        want = ref_pick(samplers, x, T, k, p)
        LIBC.srand(seed)
        rnd = LIBC.rand()
        got = H.lib.gq_hip_sample_dev(ctx.h, xd.ptr, V, T, k, p, rnd)
        assert 0 <= got < V, (got, H.lib.gq_hip_last_error(ctx.h))
        bad += got != want
    plain = T > 0 and not (0 < k < V) and p >= 1.0
    assert bad <= (1 if plain else 0), (bad, n)


def test_sample_rejects(ctx, orc):
    import guanaco_amd.hip as H
    x = ctx.upload(orc.synth_normal(3, 4096))
    assert H.lib.gq_hip_sample_dev(ctx.h, x.ptr, 4096, 1.0, 1025, 1.0, 5) == -2  # top_k above 1024
    assert H.lib.gq_hip_sample_dev(ctx.h, x.ptr, 0, 1.0, 40, 1.0, 5) == -1
    assert H.lib.gq_hip_sample_dev(ctx.h, None, 4096, 1.0, 40, 1.0, 5) == -1


def test_forward_sample_matches_reference(ctx, orc, samplers):
    """gq_hip_forward_sample: one decode step and top-k / top-p sampling on
    the device, against the same step's logits sampled by the reference."""
    import guanaco_amd.hip as H
    from guanaco_amd import spec as S
    spec, ms, pre = S.TINY_TEST, 64, 24
    dm = H.DeviceModel(ctx, spec, ms, prefill=pre)
    logits = np.empty(spec.vocab, np.float32)
    tok = 11
    for step, (T, k, p) in enumerate([(0.9, 20, 1.0), (0.8, 0, 0.8), (0.0, 0, 1.0), (1.1, 50, 1.0)]):
        pos = pre + step
        assert H.lib.gq_hip_forward_token(ctx.h, tok, pos, fptr(logits), None) >= 0
        LIBC.srand(77 + step)
        want = ref_pick(samplers, logits, T, k, p)
        LIBC.srand(77 + step)
        got = H.lib.gq_hip_forward_sample(ctx.h, tok, pos, T, k, p, LIBC.rand())
        assert got == want, (step, got, want)
        tok = got
