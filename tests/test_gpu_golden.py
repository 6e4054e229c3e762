"""The HIP path against the committed golden fixtures made from the compiled
reference (tests/golden/make_golden.py): matvec y, attention, KV slabs and
.lctx bytes, and the north-star bar on the benchmark shapes — identical
greedy tokens for 128 steps and per-layer hidden states within 1e-3
relative L2 — for the TinyLlama-shape (config 2) and Llama-3.1-8B-shape
(config 3, KV filled to 8192) models, plus the 16 largest logits of every
step, and a TinyLlama-shape variant with all weights Q8_0 whose tokens vary
from step to step."""
import os

import numpy as np
import pytest

from guanaco_amd import spec as S
from util import bits, rel_l2

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DT = {"q4_k": S.Q4_K, "q6_k": S.Q6_K, "q8_0": S.Q8_0}
MV_TOL = 1e-5     # per matvec (a correct kernel differs from the CPU order by ~1e-7)
LAYER_TOL = 1e-3  # per layer
# the 16 largest logits of each step: the median step within LOGIT_TOL
# (observed ~1e-6), every step within LOGIT_MAX.  The Q8_0 model's q and k
# entries are ~80, so its attention scores reach ~1e4, where one fp32 ulp is
# ~1e-3: at a near-tie between two positions (step 86: a top-2 gap of 0.17
# in a layer-0 head, scores of standard deviation ~3900) the GPU's and the
# CPU's summation orders move ~1e-3 of softmax weight between them, and that
# step's logits differ by 1.2e-3 with the same greedy token.  Steps without
# such a tie stay at ~1e-6.
LOGIT_TOL = 1e-5
LOGIT_MAX = 5e-3


def load(name):
    p = os.path.join(GOLD, name)
    if not os.path.exists(p):
        pytest.skip(f"{name} not generated")
    return np.load(p, allow_pickle=False)


def matvec_cases():
    g = np.load(os.path.join(GOLD, "matvec.npz"), allow_pickle=False)
    return sorted({k[:-2] for k in g.files if k.endswith("_y")})


@pytest.mark.parametrize("case", matvec_cases())
def test_matvec_vs_reference(ctx, case):
    import guanaco_amd.hip as H
    g = load("matvec.npz")
    name, shape = case.rsplit("_", 1)
    rows, cols = map(int, shape.split("x"))
    dt, seed = DT[name], int(g[case + "_seed"])
    w = ctx.synth_quant(dt, rows, cols, seed)
    x = ctx.synth_normal(cols, seed + 1)
    y = ctx.alloc(4 * rows)
    ref = g[case + "_y"]
    for path in H.MATVEC_PATHS:
        with H.matvec_path(path):
            assert H.lib.gq_hip_matvec_dev(ctx.h, dt, w.ptr, rows, cols, x.ptr, y.ptr) == 0
        out = y.download(count=rows)
        assert rel_l2(out, ref) < MV_TOL, path
        assert np.abs(out - ref).max() <= MV_TOL * (np.abs(ref).max() + 1e-30), path
    w.free(), x.free(), y.free()


@pytest.mark.parametrize("L", [512, 8192])
def test_attention_vs_golden(L):
    """K/V and q from the device generator (bit-identical to the host one the
    fixture used), attention over positions 0..L-1 of one layer."""
    import guanaco_amd.hip as H
    g = load("attention.npz")
    s = S.LLAMA8B
    c = H.Context(0)
    try:
        c.kv_init(1, s.n_kv_heads, s.head_dim, L, s.rope_theta)
        c.kv_prefill_synth(int(g[f"L{L}_seed_k"]), int(g[f"L{L}_seed_v"]), L)
        q = c.synth_normal(s.n_heads * s.head_dim, int(g[f"L{L}_seed_q"]))
        out = c.alloc(4 * s.n_heads * s.head_dim)
        assert c.attention_dev(0, L - 1, s.n_heads, q, out) == 0
        assert rel_l2(out.download(), g[f"L{L}_out"]) < MV_TOL
    finally:
        c.close()


def test_kv_append_and_lctx_vs_reference(tmp_path):
    """Device appends (with wrap) equal kv_cache_append's slabs bit for bit
    and the device .lctx save equals kv_cache_save's file byte for byte."""
    import guanaco_amd.hip as H
    g = load("kv_tiny.npz")
    nl, nkv, hd, ms = (int(v) for v in g["geometry"])
    c = H.Context(0)
    try:
        c.kv_init(nl, nkv, hd, ms, 500000.0)
        rows = g["rows"]
        for pos in range(rows.shape[2]):
            for l in range(nl):
                assert c.kv_append(l, pos, rows[0, l, pos], rows[1, l, pos]) == 0
        n = nkv * ms * hd
        for l in range(nl):
            k, v = c.kv_read_layer(l)
            assert np.array_equal(bits(k), bits(g["k"][l * n:(l + 1) * n]))
            assert np.array_equal(bits(v), bits(g["v"][l * n:(l + 1) * n]))
        path = str(tmp_path / "s.lctx")
        assert c.lctx_save(path, int(g["current_pos"]), g["tokens"]) == 0
        assert np.array_equal(np.fromfile(path, np.uint8),
                              np.fromfile(os.path.join(GOLD, "kv_tiny.lctx"), np.uint8))
    finally:
        c.close()


def run_greedy(spec, g):
    """Greedy decode on the device from the fixture's start, two ways:
    eager forward_token steps, each step's 16 largest reference logits
    compared (LOGIT_TOL) and the per-layer hidden states at every step the
    fixture holds (LAYER_TOL); then the graph-replayed decode loop.  Both
    must produce the reference's tokens at every step."""
    import guanaco_amd.hip as H
    from guanaco_amd.synth import tensor_seed
    c = H.Context(0)
    try:
        pre, ms = int(g["prefill"]), int(g["max_seq"])
        dm = H.DeviceModel(c, spec, ms, prefill=pre)
        seeds = (tensor_seed(spec.seed, -1, 13), tensor_seed(spec.seed, -1, 14))
        tokens, top_idx, top_val = g["tokens"], g["top_idx"], g["top_logits"]
        hsteps = {int(k[len("hidden_step"):]) for k in g.files if k.startswith("hidden_step")}
        n, tok = len(tokens), int(g["start_token"])
        worst_h = worst_l = 0.0
        el, eh = [], {}
        for i in range(n):
            t, logits, hid = dm.forward(tok, pre + i, want_hidden=i in hsteps)
            el.append(rel_l2(logits[top_idx[i]], top_val[i]))
            worst_l = max(worst_l, el[-1])
            if hid is not None:
                eh[i] = [rel_l2(hid[l], g[f"hidden_step{i}"][l]) for l in range(spec.n_layers)]
                worst_h = max(worst_h, max(eh[i]))
            assert t == int(tokens[i]), f"eager step {i}: token {t} vs {int(tokens[i])} (margin {g['margins'][i]:.3g})"
            tok = t
        print(f"{spec.name}: top-16 logits rel L2 per step: max {max(el):.3g} at step {int(np.argmax(el))}, "
              f"median {float(np.median(el)):.3g}, steps 0-7 {[f'{e:.2g}' for e in el[:8]]}")
        for i, e in sorted(eh.items()):
            print(f"  hidden step {i}: per-layer rel L2 {[f'{x:.2g}' for x in e]}")
        assert float(np.median(el)) < LOGIT_TOL and worst_l < LOGIT_MAX, (float(np.median(el)), worst_l)
        assert worst_h < LAYER_TOL, worst_h
        c.kv_prefill_synth(*seeds, pre)
        toks, _ = dm.decode_loop(int(g["start_token"]), pre, n, use_graph=True)
        mism = [i for i in range(n) if toks[i] != tokens[i]]
        assert not mism, f"graph: first mismatch at step {mism[0]}: {toks[mism[0]]} vs {tokens[mism[0]]}"
        print(f"{spec.name}: {n} tokens identical ({len(set(tokens.tolist()))} distinct, min margin "
              f"{float(g['margins'].min()):.3g}); top-16 logits worst rel L2 {worst_l:.3g}; hidden states "
              f"at steps {sorted(hsteps)} worst per-layer rel L2 {worst_h:.3g}")
    finally:
        c.close()


def test_tinyllama_128_greedy_steps_vs_reference():
    run_greedy(S.TINYLLAMA, load("tinyllama_greedy.npz"))


def test_tinyllama_q8_0_128_greedy_steps_vs_reference():
    """The non-degenerate variant: every weight Q8_0 (zero-mean), a different
    token at nearly every step, top-2 margins down to O(1)."""
    run_greedy(S.TINYLLAMA_Q8, load("tinyllama_q8_greedy.npz"))


def test_llama8b_128_greedy_steps_vs_reference():
    run_greedy(S.LLAMA8B, load("llama8b_greedy.npz"))
