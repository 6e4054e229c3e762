"""Decode speed of the reference's own command-line program with --device hip
(oracle/_ref/guanaco_hip: the reference, guanaco_amd/host/reference-hip.patch
and the HIP backend) on the 8B Q4_K_M shape at context 8192 — the workload
bench.py times through gq_hip_decode_loop — so the drop-in's tok/s can be set
beside bench.py's.

    python tests/cli_decode_speed.py [--dir DIR] [--tokens 128] [--check-cpu 4]

Writes DIR/llama8b.gguf (tests/golden/gguf_writer.py: bench.py's model,
spec.LLAMA8B, context 8320) and DIR/ctx8192.lctx (a session of 8192
positions of bench.py's synthetic K/V, in the .lctx format kv_cache_load
reads, session.c:107-188), then runs

    guanaco_hip --model llama8b.gguf --session ctx8192.lctx --ctx 8320
                --prompt Hello --max-tokens 128 --temperature 0 --device hip

generate() restores the session, runs the prompt at position 8192 and
decodes from there (generate.c:170-330), so the decode steps attend over
8192..8319 positions, as bench.py's do.  It prints generate()'s own decode
speed (tokens 2..N over their wall time, generate.c:333-336) and the
placement line of the HIP backend.  With --check-cpu N the same command with
--device cpu and N tokens must print the same first N tokens.

Test infrastructure (the oracle's generator writes the files); prints one
JSON line.
"""
import argparse
import ctypes as C
import json
import os
import shutil
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (ROOT, os.path.join(ROOT, "oracle"), HERE, os.path.join(HERE, "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)

import clitool  # noqa: E402
from gguf_writer import write_gguf  # noqa: E402
from guanaco_amd import spec as S  # noqa: E402
from oracle import HostKV, Oracle, fptr, u8ptr  # noqa: E402

MAX_SEQ, CTX = 8320, 8192


def write_session(path, orc, spec):
    kv = HostKV(spec.n_layers, spec.n_kv_heads, spec.head_dim, MAX_SEQ)
    kv.prefill(orc, spec, CTX)
    n = orc.lib.orc_lctx_size(C.byref(kv.s), 0)
    img = np.zeros(n, np.uint8)
    assert orc.lib.orc_lctx_write(C.byref(kv.s), CTX, None, 0, u8ptr(img), n) == 0
    img.tofile(path)
    return n


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--dir", default=None)
    ap.add_argument("--tokens", type=int, default=128)
    ap.add_argument("--check-cpu", type=int, default=0)
    a = ap.parse_args()
    d = a.dir or tempfile.mkdtemp(prefix="gq_cli_")
    os.makedirs(d, exist_ok=True)
    spec = S.LLAMA8B
    orc = Oracle()
    t0 = time.time()
    model, sess = os.path.join(d, "llama8b.gguf"), os.path.join(d, "ctx8192.lctx")
    gb = write_gguf(model, spec, MAX_SEQ, orc) / 1e9
    sb = write_session(sess, orc, spec) / 1e9
    print(f"[cli] wrote {gb:.2f} GB model and {sb:.2f} GB session in {time.time() - t0:.0f}s", flush=True)
    run_sess = os.path.join(d, "run.lctx")  # generate() saves the session back at the end (generate.c:339-344)
    kw = dict(prompt="Hello", extra=("--session", run_sess, "--ctx", str(MAX_SEQ)), threads=16, timeout=1200)
    shutil.copyfile(sess, run_sess)
    out, err = clitool.run(model, max_tokens=a.tokens, device="hip", **kw)
    assert "Session restored (pos=8192)" in out, out[-2000:]
    hip_ids = clitool.text_to_ids(clitool.generated_text(out))
    res = dict(workload="decode, llama-3.1-8b-shape-q4_k_m, ctx 8192 (session restored), greedy",
               program="oracle/_ref/guanaco_hip --device hip", tokens=len(hip_ids),
               decode_tok_s=clitool.decode_speed(out),
               placement=[l for l in err.splitlines() if l.startswith("[hip]")])
    print(f"[cli] --device hip: {res['decode_tok_s']} tok/s over {len(hip_ids)} tokens", flush=True)
    if a.check_cpu:
        shutil.copyfile(sess, run_sess)
        cpu, _ = clitool.run(model, max_tokens=a.check_cpu, device="cpu", **kw)
        cpu_ids = clitool.text_to_ids(clitool.generated_text(cpu))
        res["cpu_tokens_equal"] = cpu_ids == hip_ids[:len(cpu_ids)]
        res["cpu_decode_tok_s"] = clitool.decode_speed(cpu)
        print(f"[cli] --device cpu: first {len(cpu_ids)} tokens equal: {res['cpu_tokens_equal']}", flush=True)
    print(json.dumps(res))
    if a.dir is None:
        for f in (model, sess, run_sess):
            os.remove(f)


if __name__ == "__main__":
    main()
