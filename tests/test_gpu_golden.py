"""The HIP path against the committed golden fixtures made from the compiled
reference (tests/golden/make_golden.py): matvec y, attention, KV slabs and
.lctx bytes, and the north-star bar on the benchmark shapes — identical
greedy tokens for 128 steps and per-layer hidden states within 1e-3
relative L2 — for the TinyLlama-shape (config 2) and Llama-3.1-8B-shape
(config 3, KV filled to 8192) models, plus the 16 largest logits of every
step within 1e-3.  Besides the plain models (whose Q4_K generator makes the
token sequences degenerate) there are variants whose tokens vary from step
to step: all weights Q8_0, and the Q4_K_M mix with zero-mean Q4_K weights,
run on every matvec kernel path.  Ill-conditioned steps are also held to a
float64 evaluation of the step."""
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
# The 16 largest logits of each step: the median step within LOGIT_TOL
# (observed ~1e-6), every step within LOGIT_MAX of the reference.
LOGIT_TOL = 1e-5
LOGIT_MAX = 1e-3
# Steps where the reference's own fp32 result is F64_FLAG or more from the
# float64 evaluation of the same step (fp64_forward.py, recorded in the
# fixture) are ill conditioned, and there the device is held to the exact
# values as well, within F64_FACTOR times the reference's own distance.  The
# Q8_0 model's step 86 is one: its q and k entries reach ~80, so attention
# scores reach ~1e4, and a near-tie of two positions in a layer-0 head puts
# the reference 2.3e-4 (top-16 logits) and 6.8e-4 (hidden) from exact against
# ~2e-6 at its other steps.  The device lands as close (and 1e-6 from the
# reference) since its Q8_0 dot sums q*x on sign-extended quants; summing
# (q + 128)*x and subtracting 128*sum(x) put it 1.4e-3 / 4.4e-3 from exact.
F64_FLAG = 1e-4
F64_FACTOR = 2.0


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


def run_greedy(spec, g, paths=("auto",)):
    """Greedy decode on the device from the fixture's start.  For each matvec
    kernel path in `paths`: eager forward_token steps, each step's 16
    largest reference logits compared (LOGIT_TOL / LOGIT_MAX) and the
    per-layer hidden states at every step the fixture holds (LAYER_TOL);
    where the fixture holds a float64 evaluation of a step that the
    reference itself misses by F64_FLAG or more, the device is compared
    with the float64 values too.  Then the graph-replayed decode loop on the
    default path.  Every run must produce the reference's tokens at every
    step."""
    import guanaco_amd.hip as H
    from guanaco_amd.synth import tensor_seed
    c = H.Context(0)
    try:
        pre, ms = int(g["prefill"]), int(g["max_seq"])
        dm = H.DeviceModel(c, spec, ms, prefill=pre)
        seeds = (tensor_seed(spec.seed, -1, 13), tensor_seed(spec.seed, -1, 14))
        tokens, top_idx, top_val = g["tokens"], g["top_idx"], g["top_logits"]
        hsteps = {int(k[len("hidden_step"):]) for k in g.files if k.startswith("hidden_step")}
        f64 = {int(k[len("f64_ref_err_step"):]): g[k] for k in g.files if k.startswith("f64_ref_err_step")}
        flagged = {i for i, e in f64.items() if e[0] >= F64_FLAG or e[1] >= F64_FLAG}
        n = len(tokens)
        for path in paths:
            c.kv_prefill_synth(*seeds, pre)
            tok = int(g["start_token"])
            worst_h = worst_l = 0.0
            el, eh = [], {}
            with H.matvec_path(path):
                for i in range(n):
                    t, logits, hid = dm.forward(tok, pre + i, want_hidden=i in hsteps or i in f64)
                    got = logits[top_idx[i]]
                    el.append(rel_l2(got, top_val[i]))
                    if i in f64:
                        e_l = rel_l2(got, g[f"f64_top_logits_step{i}"])
                        e_h = max(rel_l2(hid[l], g[f"f64_hidden_step{i}"][l]) for l in range(spec.n_layers))
                        print(f"  {path} step {i} (margin {float(g['margins'][i]):.3g}): float64 distance of the "
                              f"device {e_l:.3g} / {e_h:.3g}, of the reference {f64[i][0]:.3g} / {f64[i][1]:.3g} "
                              f"(top-16 logits / hidden); device vs reference {el[-1]:.3g}")
                    if i in flagged:
                        assert e_l <= max(LOGIT_MAX, F64_FACTOR * f64[i][0]), (path, i, e_l, f64[i])
                        assert e_h <= max(LAYER_TOL, F64_FACTOR * f64[i][1]), (path, i, e_h, f64[i])
                    worst_l = max(worst_l, el[-1])
                    if i in hsteps:
                        eh[i] = [rel_l2(hid[l], g[f"hidden_step{i}"][l]) for l in range(spec.n_layers)]
                        worst_h = max(worst_h, max(eh[i]))
                    assert t == int(tokens[i]), \
                        f"{path} eager step {i}: token {t} vs {int(tokens[i])} (margin {g['margins'][i]:.3g})"
                    tok = t
            print(f"{spec.name} [{path}]: top-16 logits rel L2 per step: max {max(el):.3g} at step "
                  f"{int(np.argmax(el))}, median {float(np.median(el)):.3g}; hidden states at the recorded steps "
                  f"worst {worst_h:.3g}; ill-conditioned steps checked against float64: {sorted(flagged)}")
            for i, e in sorted(eh.items()):
                print(f"  hidden step {i}: per-layer rel L2 max {max(e):.2g}")
            assert float(np.median(el)) < LOGIT_TOL and worst_l < LOGIT_MAX, (path, float(np.median(el)), worst_l)
            assert worst_h < LAYER_TOL, (path, worst_h)
        c.kv_prefill_synth(*seeds, pre)
        toks, _ = dm.decode_loop(int(g["start_token"]), pre, n, use_graph=True)
        mism = [i for i in range(n) if toks[i] != tokens[i]]
        assert not mism, f"graph: first mismatch at step {mism[0]}: {toks[mism[0]]} vs {tokens[mism[0]]}"
        print(f"{spec.name}: {n} tokens identical on {', '.join(paths)} and in the graph loop "
              f"({len(set(tokens.tolist()))} distinct, min margin {float(g['margins'].min()):.3g}); hidden "
              f"states at steps {sorted(hsteps)}")
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


def test_tinyllama_zero_mean_q4_k_m_greedy_all_paths():
    """The TinyLlama shape with zero-mean Q4_K weights (Q4_K_M mix): tokens
    differ at nearly every step, so they discriminate on the Q4_K / Q6_K
    kernels; run on the vector-ALU, default and matrix-core matvec paths."""
    run_greedy(S.TINYLLAMA_ZM, load("tinyllama_zm_greedy.npz"), paths=("auto", "mfma", "valu"))


def test_llama8b_zero_mean_q4_k_m_greedy_all_paths():
    """The benchmark's 8B Q4_K_M shape (KV at 8192) with zero-mean Q4_K
    weights, on the default and matrix-core matvec paths."""
    run_greedy(S.LLAMA8B_ZM, load("llama8b_zm_greedy.npz"), paths=("auto", "mfma"))
