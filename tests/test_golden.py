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


def test_tinyllama_first_steps_golden(orc):
    """Two decode steps of the TinyLlama-shape model: tokens equal the
    reference's, per-layer hidden states at step 0 bit for bit."""
    g = load("tinyllama_greedy.npz")
    s = S.TINYLLAMA
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
