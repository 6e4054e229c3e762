"""The oracle against the committed golden fixtures (tests/golden/, made by
tests/golden/make_golden.py from the compiled reference in this container).
These run anywhere: the fixtures travel, the reference does not.  They pin
the oracle (and the input generator) to the reference's outputs: matvec y
bit for bit, KV slabs and .lctx bytes, whole decode steps."""
import ctypes as C
import hashlib
import os

import numpy as np
import pytest

from guanaco_amd import spec as S
from oracle import F32, HostKV, HostModel, Q4_K, Q6_K, Q8_0, fptr, u8ptr  # noqa: F401
from util import bits

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DT = {"q4_k": Q4_K, "q6_k": Q6_K, "q8_0": Q8_0}


def load(name):
    p = os.path.join(GOLD, name)
    if not os.path.exists(p):
        pytest.skip(f"{name} not generated")
    return np.load(p, allow_pickle=False)


def matvec_cases():
    g = np.load(os.path.join(GOLD, "matvec.npz"), allow_pickle=False)
    return sorted({k[:-2] for k in g.files if k.endswith("_y")})


@pytest.mark.parametrize("case", matvec_cases())
def test_matvec_golden(orc, case):
    g = load("matvec.npz")
    name, shape = case.rsplit("_", 1)
    rows, cols = map(int, shape.split("x"))
    dt, seed = DT[name], int(g[case + "_seed"])
    w = orc.synth_quant(dt, seed, rows, cols)
    assert hashlib.sha256(w.tobytes()).hexdigest() == str(g[case + "_w_sha256"]), "generator drifted"
    y = orc.matvec(dt, w, rows, cols, orc.synth_normal(seed + 1, cols))
    assert np.array_equal(bits(y), bits(g[case + "_y"]))


@pytest.mark.parametrize("L", [512, 8192])
def test_attention_golden(orc, L):
    g = load("attention.npz")
    s = S.LLAMA8B
    kv = HostKV(1, s.n_kv_heads, s.head_dim, L)
    for arr, key in ((kv.k, "seed_k"), (kv.v, "seed_v")):
        orc.lib.orc_synth_kv(C.c_uint64(int(g[f"L{L}_{key}"])), fptr(arr), 1, s.n_kv_heads, s.head_dim, L, L)
    q = orc.synth_normal(int(g[f"L{L}_seed_q"]), s.n_heads * s.head_dim)
    assert np.array_equal(bits(orc.attention(q, kv, 0, s.n_heads, L - 1)), bits(g[f"L{L}_out"]))


def test_kv_and_lctx_golden(orc):
    """20 appends on a 16-position ring (kv_cache_append) and the file
    kv_cache_save wrote: the oracle reproduces both byte for byte."""
    g = load("kv_tiny.npz")
    nl, nkv, hd, ms = (int(v) for v in g["geometry"])
    kv = HostKV(nl, nkv, hd, ms)
    rows = g["rows"]
    for pos in range(rows.shape[2]):
        for l in range(nl):
            k, v = np.ascontiguousarray(rows[0, l, pos]), np.ascontiguousarray(rows[1, l, pos])
            assert orc.lib.orc_kv_append(C.byref(kv.s), l, pos, fptr(k), fptr(v)) == 0
    assert np.array_equal(bits(kv.k), bits(g["k"])) and np.array_equal(bits(kv.v), bits(g["v"]))
    toks = np.ascontiguousarray(g["tokens"])
    n = orc.lib.orc_lctx_size(C.byref(kv.s), toks.size)
    img = np.zeros(n, np.uint8)
    assert orc.lib.orc_lctx_write(C.byref(kv.s), int(g["current_pos"]),
                                  toks.ctypes.data_as(C.POINTER(C.c_int32)), toks.size, u8ptr(img), n) == 0
    assert np.array_equal(img, np.fromfile(os.path.join(GOLD, "kv_tiny.lctx"), np.uint8))


@pytest.mark.parametrize("name,spec", [("tinyllama_greedy.npz", S.TINYLLAMA),
                                       ("tinyllama_zm_greedy.npz", S.TINYLLAMA_ZM)])
def test_tinyllama_first_steps_golden(orc, name, spec):
    """Two decode steps of the TinyLlama-shape models (the plain Q4_K
    generator and the zero-mean one): tokens equal the reference's, per-layer
    hidden states at step 0 bit for bit."""
    g = load(name)
    s = spec
    hm = HostModel(orc, s, int(g["max_seq"]))
    assert hashlib.sha256(hm.lm_head.tobytes()).hexdigest() == str(g["lm_head_sha256"])
    kv = hm.new_kv()
    pre = int(g["prefill"])
    kv.prefill(orc, s, pre)
    tok = int(g["start_token"])
    for i in range(2):
        tok, _, hid = hm.forward(kv, tok, pre + i, want_hidden=i == 0)
        assert tok == int(g["tokens"][i])
        if i == 0:
            assert np.array_equal(bits(hid), bits(g["hidden_step0"]))


def test_fp64_step_agrees_with_oracle_where_well_conditioned(orc):
    """The float64 step of tests/golden/fp64_forward.py against the fp32
    oracle on the tiny model: ~1e-6 apart, so it computes the same function
    (a dropped term, a wrong index or sign would show as O(1))."""
    from fp64_forward import forward_step
    s, ms, pre = S.TINY_ZM, 64, 24
    hm = HostModel(orc, s, ms)
    kv = hm.new_kv()
    kv.prefill(orc, s, pre)
    tok = 11
    for i in range(3):
        l64, h64 = forward_step(hm, kv, tok, pre + i)
        tok, l32, h32 = hm.forward(kv, tok, pre + i, want_hidden=True)
        assert np.linalg.norm(l32 - l64) / np.linalg.norm(l64) < 1e-5
        for l in range(s.n_layers):
            assert np.linalg.norm(h32[l] - h64[l]) / np.linalg.norm(h64[l]) < 1e-5
        assert int(np.argmax(l64)) == tok


def test_zero_mean_q4k_generator(orc):
    """gq_q4k_zm_byte: every sub-block's min equals its scale and dmin is
    fp16(7.5 d), so each row of weights sums to about zero (the plain
    generator's rows sum to ~5 per weight)."""
    from util import dequant_q4k_f64
    zm = orc.synth_quant(S.Q4_K | S.SYNTH_Q4K_ZERO_MEAN, 3, 256, 1024)
    blk = zm.reshape(256, 4, 144)
    d = blk[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dmin = blk[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    assert np.array_equal(dmin, (7.5 * d).astype(np.float16).astype(np.float64))
    w = dequant_q4k_f64(zm, 256, 1024)
    w0 = dequant_q4k_f64(orc.synth_quant(S.Q4_K, 3, 256, 1024), 256, 1024)
    assert abs(w.mean()) < 0.05 * w.std() and w0.mean() > 0.5 * w0.std()
    # the scales unpack (get_scale_min_k4) to sc_j == m_j: the mean of each
    # 32-weight sub-block is d*sc*(mean(q) - 7.5), zero in expectation
    sub = w.reshape(256, 4, 8, 32)
    assert np.abs(sub.mean(axis=(0, 3))).max() < 0.1 * w.std()
