"""Decode benchmark: Llama-3.1-8B-shape Q4_K_M, KV pre-filled to 8192.

One "step" is one greedy decode token through the whole model on the GPU
(embedding, 32 layers, final norm, LM head, argmax), replayed from a captured
HIP graph; weights (4.6 GB, synthetic, generated in HBM from seeds) and the
KV cache are resident before the timed region.  Steps start at position
8192 (warm-up steps are run from the same position first and overwritten).

Prints ONE JSON line.  value = tokens/s over exactly --steps tokens between
two device synchronisations.  roofline = the dominant matvec (the fused
gate/up + SwiGLU launch, the int8 matrix-core kernel mvm_kernel<Q4_K,
MV_SWIGLU> on tile-interleaved weights): its algorithmic bytes per launch
over its average duration, measured live with HIP events around 64
back-to-back launches cycling over the 32 layers at the same position;
traffic = its HBM bytes per launch from the committed rocprofv3 counter runs
(profiles/mvm_gate_up_llama8b_hbm_traffic.md).  cpu_baseline =
the reference's own CPU forward() (oracle/_ref/libref.so) timed on this
host on a bounded sample, or the oracle port when the reference build is
absent.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
CTX = 8192


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "mvm_gate_up_llama8b_hbm_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the gate/up kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs (scaled by a copy kernel of known
    size; the file gives the commands), or None when that file is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def cpu_baseline(spec, seconds=20.0, threads=8):
    """Reference forward() on the 8B shape at pos 8192, a bounded number of
    tokens (~`seconds` of CPU work)."""
    import ctypes as C
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import HostModel, Oracle, Ref, RefModel, ref_available

    orc = Oracle(threads=min(os.cpu_count() or 1, 16))
    t0 = time.time()
    hm = HostModel(orc, spec, CTX + 8)
    kv = hm.new_kv()
    kv.prefill(orc, spec, CTX)
    log(f"cpu baseline: host model built in {time.time() - t0:.1f}s")
    kind = "reference" if ref_available() else "port"
    if kind == "reference":
        ref = Ref(threads=threads)
        rm = RefModel(ref, hm)
        rm.load_kv(kv)
        del kv
        step = lambda tok, pos: rm.forward(tok, pos)[0]  # noqa: E731
    else:
        orc.set_threads(threads)
        orc.set_faithful(True)
        step = lambda tok, pos: hm.forward(kv, tok, pos)[0]  # noqa: E731
    tok, n, t0 = 1, 0, time.time()
    while True:
        tok = step(tok, CTX + n)
        n += 1
        if time.time() - t0 > seconds or n >= 8:
            break
    dt = time.time() - t0
    return {"value": n / dt, "unit": "tok/s", "cores": threads, "kind": kind,
            "sample": f"{n} greedy decode tokens of the same 8B-shape Q4_K_M model at positions "
                      f"{CTX}..{CTX + n - 1} through the reference CPU forward() "
                      f"({'compiled reference' if kind == 'reference' else 'C restatement'}, "
                      f"{threads} threads, Q6_K/Q8_0 single-threaded as in the reference)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--eager", action="store_true", help="no HIP graph (diagnostics)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is design-only, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import guanaco_amd.hip as H
    from guanaco_amd import spec as S

    spec = S.LLAMA8B
    max_seq = max(CTX + max(args.steps, args.warmup, 128), 8320)
    max_seq = (max_seq + 63) // 64 * 64
    ctx = H.Context(0)
    n_cu, arch = ctx.info()
    t0 = time.time()
    dm = H.DeviceModel(ctx, spec, max_seq, prefill=CTX)
    ctx.sync()
    log(f"model + KV generated on device in {time.time() - t0:.1f}s ({arch}, {n_cu} CUs)")

    start_tok = 128000 % spec.vocab
    if args.warmup:
        dm.decode_loop(start_tok, CTX, args.warmup, use_graph=not args.eager)
    ctx.sync()
    t0 = time.perf_counter()
    toks, dev_ms = dm.decode_loop(start_tok, CTX, args.steps, use_graph=not args.eager)
    ctx.sync()
    wall = time.perf_counter() - t0
    tok_s = args.steps / wall
    log(f"{args.steps} steps in {wall * 1e3:.1f} ms (device {dev_ms:.1f} ms); tokens {list(toks[:8])}...")

    # per-kernel-class device time of one eager step at the first timed position
    prof = dm.profile_step(start_tok, CTX)
    # the dominant matvec: the fused gate/up + SwiGLU launch (one per layer,
    # mvm_kernel<Q4_K, MV_SWIGLU>); algorithmic bytes per launch =
    # 2 x 14336 x 4096 Q4_K weights (144 B per 256) + x, norm weight, output
    gu = prof["gate_up"]
    bytes_per_launch = gu["bytes"] / max(gu["launches"], 1)
    # its average launch duration: back-to-back launches over all 32 layers
    # between two HIP events on the stream the kernels run on
    op_ms = {op: round(dm.time_op(op, CTX, 64 if op != "lm_head" else 8), 5)
             for op in H.CLASS_NAMES if op != "other"}
    avg_ms = op_ms["gate_up"]
    achieved = bytes_per_launch / (avg_ms * 1e-3) / 1e9
    log(f"back-to-back ms per launch: {json.dumps(op_ms)}")
    classes = {k: {"ms": round(v["ms"], 4), "launches": v["launches"],
                   "GB_per_s": round(v["bytes"] / max(v["ms"], 1e-9) / 1e6, 1)}
               for k, v in prof.items() if v["launches"]}
    step_ms = sum(v["ms"] for v in prof.values())
    log(f"profile (eager step): {json.dumps(classes)}")

    weight_bytes = spec.weight_bytes_per_token()
    kv_bytes = spec.kv_bytes_per_token(CTX)
    out = {
        "metric": "decode tok/s, Llama-3.1-8B-shape Q4_K_M, ctx 8192; matvec GB/s vs HBM peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k/q6_k weights, fp32 activations and KV",
        "data": "synthetic (seeded random-init weights and N(0,1) KV, generated in HBM)",
        "config": {"workload": "configs[2]: Llama-3.1-8B-shape Q4_K_M decode, KV filled to 8192, "
                               "greedy steps from pos 8192",
                   "model": spec.name, "global_batch": 1, "seq_len": CTX, "parallelism": "none (1 GPU)",
                   "max_seq": max_seq, "graph": not args.eager},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "kernel": "mvm_kernel<Q4_K, MV_SWIGLU> (gate/up + SwiGLU on the int8 matrix cores, "
                               "one launch per layer)",
                     "avg_launch_ms": round(avg_ms, 5), "bytes_per_launch": int(bytes_per_launch)},
        "per_token": {"weight_bytes": weight_bytes, "kv_bytes_at_8192": kv_bytes,
                      "effective_GB_per_s": round((weight_bytes + kv_bytes) * tok_s / 1e9, 1),
                      "eager_step_kernel_ms": round(step_ms, 4), "classes": classes,
                      "op_ms_back_to_back": op_ms},
        "device": {"arch": arch, "cus": n_cu},
    }
    ctx.close()
    if not args.no_cpu:
        try:
            out["cpu_baseline"] = cpu_baseline(spec, args.cpu_seconds)
        except Exception as e:  # the GPU number stands; say why the CPU leg is missing
            out["cpu_baseline"] = {"value": None, "error": repr(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
