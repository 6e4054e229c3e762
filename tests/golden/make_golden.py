"""Generate the golden fixtures of tests/golden/ from the compiled reference.

Runs only where oracle/_ref/libref.so is built from /root/reference's own
sources (oracle/Makefile); the fixtures it writes are small data files that
travel with the repository (the reference itself never does).

    python tests/golden/make_golden.py [--skip-8b]

What comes from where (the README next to this script says the same):
  matvec.npz          y = W x from the reference's matvec_q4k/q6k/q8_0_f32
  attention.npz       the oracle's attention (pinned to the reference through
                      test_forward_bitexact_vs_reference: whole-step logits)
  kv_tiny.npz/.lctx   slabs after kv_cache_append (with wrap) and the file
                      kv_cache_save writes, from the reference
  tinyllama_greedy.npz / tinyllama_q8_greedy.npz / tinyllama_zm_greedy.npz /
  llama8b_greedy.npz / llama8b_zm_greedy.npz
                      greedy tokens, top-2 logit margins and the 16 largest
                      logits (indices and values) of every step from the
                      reference's forward() + sample_greedy; per-layer hidden
                      states at steps 0, 63, 127 and the smallest-margin
                      steps from the oracle, run in lock step (its logits are
                      asserted bit-identical to the reference's at every
                      step); at a few of those steps the same step in float64
                      (fp64_forward.py) and the reference's distance from it
Inputs are the deterministic generator of guanaco_amd/csrc/gq_synth.h
(GENERATOR_VERSION below); each file records seeds and SHA-256 of weights.
"""
import argparse
import ctypes as C
import hashlib
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, HERE)

from guanaco_amd import spec as S  # noqa: E402
from oracle import (Q4_K, Q6_K, Q8_0, F32, HostKV, HostModel, Oracle, Ref, RefModel,  # noqa: E402
                    RModelConfig, rtensor)

GENERATOR_VERSION = 1
MATVEC_CASES = [(Q4_K, 1, 256), (Q4_K, 8, 512), (Q4_K, 64, 1024), (Q4_K, 4096, 4096),
                (Q6_K, 1, 256), (Q6_K, 8, 512), (Q6_K, 64, 1024),
                (Q8_0, 1, 256), (Q8_0, 8, 512), (Q8_0, 64, 1024)]
NAMES = {Q4_K: "q4_k", Q6_K: "q6_k", Q8_0: "q8_0"}
TOPK = 16  # reference logits recorded per greedy step (largest first)


def log(m):
    print(f"[golden] {m}", flush=True)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def matvec_seed(dt, rows, cols):
    return 0x60D0000 + (dt << 20) + (rows << 8) + cols


def make_matvec(orc, ref):
    out = {"generator_version": np.int64(GENERATOR_VERSION)}
    for dt, rows, cols in MATVEC_CASES:
        seed = matvec_seed(dt, rows, cols)
        w = orc.synth_quant(dt, seed, rows, cols)
        x = orc.synth_normal(seed + 1, cols)
        y = ref.matvec(dt, w, rows, cols, x)
        key = f"{NAMES[dt]}_{rows}x{cols}"
        out[key + "_seed"] = np.int64(seed)
        out[key + "_w_sha256"] = np.array(sha(w))
        out[key + "_y"] = y
    np.savez(os.path.join(HERE, "matvec.npz"), **out)
    log(f"matvec: {len(MATVEC_CASES)} cases")


def make_attention(orc):
    out = {"generator_version": np.int64(GENERATOR_VERSION)}
    s = S.LLAMA8B
    for L in (512, 8192):
        kv = HostKV(1, s.n_kv_heads, s.head_dim, L)
        seed_k, seed_v = 0xA77E0 + L, 0xA77E1 + L
        for arr, sd in ((kv.k, seed_k), (kv.v, seed_v)):
            orc.lib.orc_synth_kv(C.c_uint64(sd), arr.ctypes.data_as(C.POINTER(C.c_float)), 1,
                                 s.n_kv_heads, s.head_dim, L, L)
        q = orc.synth_normal(0xA77E2 + L, s.n_heads * s.head_dim)
        o = orc.attention(q, kv, 0, s.n_heads, L - 1)
        out[f"L{L}_seed_k"], out[f"L{L}_seed_v"] = np.int64(seed_k), np.int64(seed_v)
        out[f"L{L}_seed_q"] = np.int64(0xA77E2 + L)
        out[f"L{L}_out"] = o
    np.savez(os.path.join(HERE, "attention.npz"), **out)
    log("attention: L 512, 8192")


def make_kv_tiny(orc, ref):
    """2 layers x 2 kv heads x 16 positions x hd 8: appends at positions
    0..19 (16..19 wrap onto 0..3), then kv_cache_save with 20 tokens."""
    nl, nkv, hd, ms = 2, 2, 8, 16
    cfg = RModelConfig(nkv * hd, nkv, nkv, hd, nl, 100, 1, 2, 64, ms, None, None)
    arena = ref.lib.arena_create(1 << 20)
    kvp = ref.lib.kv_cache_create(arena, C.byref(cfg), ms)
    rows = orc.synth_normal(0x7171, 2 * nl * 20 * nkv * hd).reshape(2, nl, 20, nkv * hd)
    keep = []
    for pos in range(20):
        for l in range(nl):
            tk = rtensor(rows[0, l, pos], F32, (nkv, hd))
            tv = rtensor(rows[1, l, pos], F32, (nkv, hd))
            keep += [tk, tv]
            assert ref.lib.kv_cache_append(kvp, l, C.byref(tk), C.byref(tv), pos) == 0
    n = nkv * ms * hd
    k = np.concatenate([np.ctypeslib.as_array(C.cast(ref.lib.kv_cache_raw_k(kvp, l), C.POINTER(C.c_float)),
                                              shape=(n,)).copy() for l in range(nl)])
    v = np.concatenate([np.ctypeslib.as_array(C.cast(ref.lib.kv_cache_raw_v(kvp, l), C.POINTER(C.c_float)),
                                              shape=(n,)).copy() for l in range(nl)])
    toks = (C.c_int * 20)(*range(100, 120))
    path = os.path.join(HERE, "kv_tiny.lctx")
    assert ref.lib.kv_cache_save(kvp, C.byref(cfg), ms, 20, toks, 20, path.encode()) == 0
    np.savez(os.path.join(HERE, "kv_tiny.npz"), generator_version=np.int64(GENERATOR_VERSION),
             geometry=np.array([nl, nkv, hd, ms], np.int32), rows_seed=np.int64(0x7171), rows=rows,
             k=k, v=v, tokens=np.arange(100, 120, dtype=np.int32), current_pos=np.int32(20))
    ref.lib.arena_destroy(arena)
    log("kv_tiny: 20 appends, .lctx")


def make_greedy(orc, ref, spec, max_seq, prefill, start, steps, name, hidden_steps=(0, 63, 127), n_low=0,
                extra=(), n_f64_low=0):
    """128 greedy steps of the reference's forward() + sample_greedy with the
    oracle in lock step (its logits asserted bit-identical at every step).
    Per-layer hidden states are kept for `hidden_steps`, `extra` and the
    n_low steps with the smallest top-2 margins.  For the n_f64_low
    smallest-margin steps and `extra`, the step is also run in float64
    (fp64_forward.py) on the reference's own cache, and the fixture records
    the exact top-16 logits and hidden states and how far the reference's
    fp32 result is from them."""
    from fp64_forward import forward_step
    t0 = time.time()
    hm = HostModel(orc, spec, max_seq)
    kv = hm.new_kv()
    kv.prefill(orc, spec, prefill)
    rm = RefModel(ref, hm)
    rm.load_kv(kv)
    log(f"{name}: model built in {time.time() - t0:.0f}s")
    toks, margins, hid_all, top_idx, top_val, inputs = [], [], [], [], [], []
    tok = start
    for i in range(steps):
        pos = prefill + i
        inputs.append(tok)
        t_ref, logits = rm.forward(tok, pos)
        top2 = np.sort(logits)[-2:]
        margins.append(float(top2[1] - top2[0]))
        idx = np.argsort(logits, kind="stable")[::-1][:TOPK]
        top_idx.append(idx.astype(np.int32))
        top_val.append(logits[idx].astype(np.float32))
        t_orc, l_orc, hid = hm.forward(kv, tok, pos, want_hidden=True)
        assert t_orc == t_ref and np.array_equal(l_orc.view(np.uint32), logits.view(np.uint32)), \
            f"{name}: oracle and reference differ at step {i}"
        hid_all.append(hid.copy())
        toks.append(t_ref)
        tok = t_ref
        if i % 16 == 0:
            log(f"{name}: step {i} token {t_ref} margin {margins[-1]:.4g} ({time.time() - t0:.0f}s)")
    order = [int(i) for i in np.argsort(margins, kind="stable")]
    keep_h = sorted(set(hidden_steps) | set(extra) | set(order[:n_low]))
    f64_steps = sorted(set(extra) | set(order[:n_f64_low]))
    out = dict(generator_version=np.int64(GENERATOR_VERSION), model_seed=np.int64(spec.seed),
               start_token=np.int32(start), prefill=np.int32(prefill), max_seq=np.int32(max_seq),
               tokens=np.array(toks, np.int32), margins=np.array(margins, np.float32),
               top_idx=np.stack(top_idx), top_logits=np.stack(top_val),
               embed_sha256=np.array(sha(hm.embed)), lm_head_sha256=np.array(sha(hm.lm_head)))
    for i in keep_h:
        out[f"hidden_step{i}"] = hid_all[i]
    # every step reads cache rows 0..pos only, so the final cache serves them all
    for i in f64_steps:
        l64, h64 = forward_step(hm, kv, inputs[i], prefill + i)
        out[f"f64_top_logits_step{i}"] = l64[top_idx[i]]
        out[f"f64_hidden_step{i}"] = h64.astype(np.float32)
        e_l = float(np.linalg.norm(top_val[i] - l64[top_idx[i]]) / np.linalg.norm(l64[top_idx[i]]))
        e_h = max(float(np.linalg.norm(hid_all[i][l] - h64[l]) / np.linalg.norm(h64[l]))
                  for l in range(spec.n_layers))
        out[f"f64_ref_err_step{i}"] = np.array([e_l, e_h], np.float64)
        log(f"{name}: step {i} (margin {margins[i]:.4g}) reference vs float64: top-16 logits {e_l:.3g}, "
            f"hidden per layer {e_h:.3g} ({time.time() - t0:.0f}s)")
    np.savez(os.path.join(HERE, f"{name}.npz"), **out)
    rm.close()
    log(f"{name}: {steps} steps in {time.time() - t0:.0f}s; {len(set(toks))} distinct tokens; "
        f"min margin {min(margins):.4g}; hidden states at {keep_h}; float64 at {f64_steps}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--skip-8b", action="store_true")
    ap.add_argument("--only", default="")
    a = ap.parse_args()
    orc = Oracle(threads=8)
    orc.set_faithful(False)  # threads over rows only: per-row order unchanged
    ref = Ref(threads=8)
    only = set(a.only.split(",")) if a.only else None
    if not only or "matvec" in only:
        make_matvec(orc, ref)
    if not only or "attention" in only:
        make_attention(orc)
    if not only or "kv" in only:
        make_kv_tiny(orc, ref)
    if not only or "tinyllama" in only:
        make_greedy(orc, ref, S.TINYLLAMA, 640, 512, 1, 128, "tinyllama_greedy")
    if not only or "tinyllama_q8" in only:
        # step 86 has a near-tie of two attention positions at scores ~1e4
        make_greedy(orc, ref, S.TINYLLAMA_Q8, 640, 512, 1, 128, "tinyllama_q8_greedy", n_low=4, extra=(86,),
                    n_f64_low=1)
    if not only or "tinyllama_zm" in only:
        make_greedy(orc, ref, S.TINYLLAMA_ZM, 640, 512, 1, 128, "tinyllama_zm_greedy", n_low=8, n_f64_low=3)
    if (not only or "llama8b" in only) and not a.skip_8b:
        make_greedy(orc, ref, S.LLAMA8B, 8320, 8192, 128000, 128, "llama8b_greedy")
    if (not only or "llama8b_zm" in only) and not a.skip_8b:
        make_greedy(orc, ref, S.LLAMA8B_ZM, 8320, 8192, 128000, 128, "llama8b_zm_greedy", n_low=5, n_f64_low=1)


if __name__ == "__main__":
    main()
