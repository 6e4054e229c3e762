"""Decode benchmark: Llama-3.1-8B-shape Q4_K_M, KV pre-filled to 8192.

One "step" is one greedy decode token through the whole model on the GPU
(embedding, 32 layers, final norm, LM head, argmax), replayed from a captured
HIP graph; weights (4.6 GB, synthetic, generated in HBM from seeds) and the
KV cache are resident before the timed region.  Steps start at position
8192 (warm-up steps are run from the same position first and overwritten).

Prints ONE JSON line.  value = tokens/s over exactly --steps tokens between
two device synchronisations.

roofline = the op class that takes the largest share of the step (at ctx
8192: attention, the split-K partial kernel and its merge, one pair per
layer): its algorithmic bytes per launch (K and V of every position, q and
the output) over its average duration, measured live with HIP events around
64 back-to-back launches cycling over the 32 layers at the same position, on
the stream the kernels run on.  roofline_classes gives the same figures for
every op class, with each class's share of the step.  traffic = HBM bytes
per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs
(profiles/decode_llama8b_ctx8192_hbm_traffic.md, which gives the commands
and the copy-kernel scaling).

cpu_baseline = the reference's own CPU forward() (oracle/_ref/libref.so, or
the oracle's C restatement when that build is absent) on this host: the
median of 5 timed greedy tokens at nproc threads (the headline) and at 8,
plus the reference's Q4_K, Q6_K and Q8_0 matvec GB/s on the down-projection
shape (median over a rotation of ~1.5 GB of distinct matrices per dtype, so
every call reads DRAM), and what lscpu and /proc/meminfo say of the host.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
CTX = 8192

# the kernels behind each op class at the 8B shape (layers whose v and down
# are Q6_K alternate with all-Q4_K layers)
CLASS_KERNELS = {
    "qkv": "mvx_pair_kernel (Q4_K q/k + Q6_K v) / mvx_kernel<Q4_K, STORE> (q/k/v): RMSNorm, "
           "RoPE and K/V append fused, x * w shared in LDS",
    "attention": "attn_partial32_kernel<128, 4> + attn_merge_kernel (split-K partials over 32-position "
                 "chunks, merge)",
    "o_proj": "mvx_kernel<Q4_K, RESID> (o + residual, x shared in LDS)",
    "gate_up": "mvm_kernel<Q4_K, SWIGLU> (int8 matrix cores, RMSNorm + SwiGLU fused)",
    "down": "mvx_kernel<Q6_K in the unit layout / Q4_K, RESID> (down + residual)",
    "lm_head": "mvm_kernel<Q6_K, STORE> (int8 matrix cores, final RMSNorm fused, no per-stage barrier)",
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_llama8b_ctx8192_hbm_traffic.md")


def measured_traffic():
    """HBM bytes per launch of each op class, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE runs (scaled by a copy kernel of known size; the
    file gives the commands): {class: bytes}, empty when the file is absent."""
    out = {}
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch[") and "]:" in line:
                    k, v = line[len("traffic_bytes_per_launch["):].split("]:", 1)
                    out[k.strip()] = int(v.strip())
    except OSError:
        pass
    return out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def host_info():
    """What the host tells about its CPUs and memory (lscpu, /proc/meminfo,
    the NUMA nodes and the last-level cache): no root is needed for any of it."""
    import subprocess
    info = {"cpu": cpu_model()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        want = ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core", "CPU(s)",
                "NUMA node(s)", "L3 cache", "CPU max MHz")
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in want:
                info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemTotal"):
                    info["MemTotal"] = line.split(":", 1)[1].strip()
    except OSError:
        pass
    try:
        info["numa_nodes"] = len([d for d in os.listdir("/sys/devices/system/node") if d.startswith("node")])
    except OSError:
        pass
    try:
        with open("/sys/devices/system/cpu/cpu0/cache/index3/size") as f:
            info["L3_per_cpu0_domain"] = f.read().strip()
    except OSError:
        pass
    info["affinity_cpus"] = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None
    return info


def cpu_baseline(spec, n_tok=5):
    """The reference's CPU forward() on the 8B shape at pos 8192: n_tok timed
    greedy tokens (after one untimed) at nproc threads and at 8, and its
    Q4_K / Q6_K matvec on the down-projection shape (4096 x 14336)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import HostModel, Oracle, Ref, RefModel, ref_available
    from guanaco_amd import spec as S

    nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    orc = Oracle(threads=min(nproc, 16))
    t0 = time.time()
    hm = HostModel(orc, spec, CTX + 8)
    kv = hm.new_kv()
    kv.prefill(orc, spec, CTX)
    log(f"cpu baseline: host model built in {time.time() - t0:.1f}s")
    kind = "reference" if ref_available() else "port"
    rows, cols = spec.hidden, spec.ff
    x = orc.synth_normal(7, cols)
    # matvec inputs rotated over ~1.5 GB per dtype, far past any host's L3,
    # so each call streams its weights from DRAM
    mats = {}
    for dt in (S.Q4_K, S.Q6_K, S.Q8_0):
        n = max(2, int(1.5e9 // S.qbytes(dt, rows, cols)))
        mats[dt] = [orc.synth_quant(dt, 99 + i, rows, cols) for i in range(n)]
    log(f"cpu baseline: {sum(len(v) for v in mats.values())} matvec inputs in "
        f"{sum(w.nbytes for v in mats.values() for w in v) / 1e9:.1f} GB")
    runs = {}
    for threads in sorted({nproc, 8}, reverse=True):
        if kind == "reference":
            ref = Ref(threads=threads)
            rm = RefModel(ref, hm)
            rm.load_kv(kv)
            step = lambda tok, pos: rm.forward(tok, pos)[0]  # noqa: E731
            mv = ref.matvec
        else:
            orc.set_threads(threads)
            orc.set_faithful(True)
            step = lambda tok, pos: hm.forward(kv, tok, pos)[0]  # noqa: E731
            mv = orc.matvec
        tok = step(1, CTX)  # untimed: first touch of the weights
        dts = []
        for n in range(n_tok):
            t1 = time.perf_counter()
            tok = step(tok, CTX + 1 + n)
            dts.append(time.perf_counter() - t1)
        gbs = {}
        for dt, ws in mats.items():
            ts = []
            for w in ws:  # each call on a matrix the previous ones evicted from the caches
                t1 = time.perf_counter()
                mv(dt, w, rows, cols, x)
                ts.append(time.perf_counter() - t1)
            gbs[S.DTYPE_NAME[dt]] = round((ws[0].nbytes + 4 * (rows + cols)) / statistics.median(ts) / 1e9, 2)
        runs[threads] = {"tok_s": round(1.0 / statistics.median(dts), 4),
                         "tok_s_each": [round(1.0 / d, 4) for d in dts],
                         "matvec_GB_per_s": gbs}
        log(f"cpu baseline, {threads} threads: {json.dumps(runs[threads])}")
        if kind == "reference":
            rm.close()
    head = runs[nproc]
    return {"value": head["tok_s"], "unit": "tok/s", "cores": nproc, "kind": kind,
            "cpu": cpu_model(), "nproc": nproc, "host": host_info(),
            "runs": {str(k): v for k, v in runs.items()},
            "sample": f"median of {n_tok} greedy decode tokens (after one untimed) of the same 8B-shape "
                      f"Q4_K_M model at positions {CTX + 1}..{CTX + n_tok} through the reference CPU "
                      f"forward() ({'compiled reference' if kind == 'reference' else 'C restatement'}), "
                      f"at nproc = {nproc} threads (value) and at 8 (runs); Q6_K and Q8_0 matvecs are "
                      f"single-threaded in the reference.  matvec_GB_per_s: the reference's Q4_K, Q6_K and "
                      f"Q8_0 matvec on {rows} x {cols}, the median over a rotation of ~1.5 GB of distinct "
                      f"matrices per dtype (each call from DRAM, not the L3)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-tokens", type=int, default=5, help="timed CPU tokens per thread count")
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

    # per-kernel-class device time and algorithmic bytes of one eager step at
    # the first timed position
    prof = dm.profile_step(start_tok, CTX)
    # every class's average launch duration: back-to-back launches over all
    # 32 layers between two HIP events on the stream the kernels run on
    op_ms = {op: round(dm.time_op(op, CTX, 64 if op != "lm_head" else 8), 5)
             for op in H.CLASS_NAMES if op != "other"}
    log(f"back-to-back ms per launch: {json.dumps(op_ms)}")
    traffic = measured_traffic()
    roof = []
    for op, ms in op_ms.items():
        c = prof[op]
        n = max(c["launches"], 1)
        b = c["bytes"] / n
        gbs = b / (ms * 1e-3) / 1e9
        roof.append({"class": op, "kernels": CLASS_KERNELS[op], "bytes_per_launch": int(b),
                     "avg_launch_ms": ms, "achieved_GB_per_s": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "launches_per_step": c["launches"],
                     "ms_per_step": round(ms * c["launches"], 4), "traffic": traffic.get(op)})
    dom = max(roof, key=lambda r: r["ms_per_step"])
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
        "roofline": {"bound": "hbm", "achieved": dom["achieved_GB_per_s"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": dom["frac"], "traffic": dom["traffic"],
                     "kernel": f"{dom['class']}: {dom['kernels']}, one launch per layer",
                     "avg_launch_ms": dom["avg_launch_ms"], "bytes_per_launch": dom["bytes_per_launch"],
                     "step_share": round(dom["ms_per_step"] / sum(r["ms_per_step"] for r in roof), 4)},
        "roofline_classes": roof,
        "per_token": {"weight_bytes": weight_bytes, "kv_bytes_at_8192": kv_bytes,
                      "effective_GB_per_s": round((weight_bytes + kv_bytes) * tok_s / 1e9, 1),
                      "eager_step_kernel_ms": round(step_ms, 4), "classes": classes,
                      "op_ms_back_to_back": op_ms},
        "device": {"arch": arch, "cus": n_cu},
    }
    ctx.close()
    if not args.no_cpu:
        try:
            out["cpu_baseline"] = cpu_baseline(spec, args.cpu_tokens)
        except Exception as e:  # the GPU number stands; say why the CPU leg is missing
            out["cpu_baseline"] = {"value": None, "error": repr(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
