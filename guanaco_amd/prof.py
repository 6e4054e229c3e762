"""Workloads for rocprofv3 runs (the commands recorded under profiles/).

    python3 -m guanaco_amd.prof copy --mib 256 --iters 20
        the plain copy kernel (gq_hip_copy_dev) on a buffer of known size:
        the reference that scales the FETCH_SIZE / WRITE_SIZE counters into
        HBM bytes (expected per dispatch: mib MiB read and mib MiB written).

    python3 -m guanaco_amd.prof configs
        the benchmark configs other than the headline one, with synthetic
        inputs generated on the device: (1) one Q4_K 4096x4096 matvec
        rotating over 48 matrices (> the 256 MB MALL); (2) TinyLlama-shape
        greedy decode, 128 steps from a 512-position KV prefix; (4) split-K
        attention per layer at 8192 / 16384 / 32768 positions on the 8B shape
        (cycling over the 32 layers' caches) and a .lctx restore of a
        4096-token prefix (1 GiB of K/V) from pinned host memory.  Prints one
        JSON line per result.

    python3 -m guanaco_amd.prof gemm --dtype 4 --rows 4096 --cols 4096 --tokens 512 --iters 20
        one prefill GEMM shape launched back to back (for counter runs).

    python3 -m guanaco_amd.prof config5
        the prefill chunk on the 8B shape: the bf16-MFMA GEMM of 512 tokens
        against each projection shape (4096x4096, 1024x4096, 14336x4096 and
        the 4096x14336 down projection, Q4_K and Q6_K), RoPE + append +
        causal attention of the 512 tokens, and forward() of a 512-token
        prompt through the whole 32-layer model.

    python3 -m guanaco_amd.prof upload
        the 8B shape's 4.6 GB of weights uploaded tensor by tensor from
        pageable host memory (gq_hip_upload_weight's pinned staging): GB/s,
        and hipMemGetInfo before, while resident and after gq_hip_destroy.

    python3 -m guanaco_amd.prof floor --iters 64
        a read-only streaming kernel (gq_hip_time_read) launched once per size
        over a 2 GiB buffer: the time one launch needs just to read the bytes
        each decode kernel moves, and a 1-512 MiB sweep.

    python3 -m guanaco_amd.prof sample --vocab 128256 --iters 50
        on-device sampling (gq_hip_sample_dev) of N(0, 3^2) logits already
        in HBM: greedy, top-k 40, top-p 0.9 and plain temperature, each the
        wall time per call including the 4-byte token copy back.

The decode workload itself is ``python3 bench.py --eager`` (one kernel launch
per op, so per-dispatch counters map onto ops).
"""
import argparse
import ctypes as C
import json
import os
import tempfile
import time

import numpy as np

from . import hip as H
from . import spec as S


def run_copy(mib, iters):
    ctx = H.Context(0)
    n = mib << 20
    src, dst = ctx.alloc(n), ctx.alloc(n)
    for _ in range(iters):
        ctx.check(H.lib.gq_hip_copy_dev(ctx.h, dst.ptr, src.ptr, n), "copy")
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(iters):
        ctx.check(H.lib.gq_hip_copy_dev(ctx.h, dst.ptr, src.ptr, n), "copy")
    ctx.sync()
    dt = (time.perf_counter() - t0) / iters
    print(f"copy {mib} MiB: {dt * 1e6:.1f} us per launch, {2 * n / dt / 1e9:.0f} GB/s (read + write)", flush=True)
    ctx.close()


def emit(**kw):
    print(json.dumps(kw), flush=True)


# algorithmic bytes per launch of the decode step's kernels on the 8B shape at
# ctx 8192 (the figures bench.py's roofline uses)
DECODE_BYTES = [("q/k/v (even layers)", 15278080), ("q/k/v (odd layers)", 14196736), ("o", 9486336),
                ("gate/up", 66134016), ("down Q6_K", 48259072), ("down Q4_K", 33120256),
                ("attention K/V at ctx 8192", 67133440), ("LM head", 431408128)]


def run_floor(iters):
    """One launch of the read-only streaming kernel per size, rotating over
    a 2 GiB buffer so that every launch reads HBM (up to 128 regions, each
    2 MiB-aligned): the time a single launch needs just to read that many
    bytes, at the decode kernels' sizes and on a sweep."""
    ctx = H.Context(0)
    span = 2 << 30
    buf = ctx.alloc(span)
    sizes = [(name, b) for name, b in DECODE_BYTES]
    sizes += [(f"{m} MiB", m << 20) for m in (1, 2, 4, 8, 16, 32, 64, 128, 256, 512)]
    for name, b in sizes:
        b16 = (b + 15) // 16 * 16
        stride = (b16 + (2 << 20) - 1) // (2 << 20) * (2 << 20)
        n_buf = max(1, min(128, span // stride))
        ms = H.lib.gq_hip_time_read(ctx.h, buf.ptr, b16, stride, n_buf, iters)
        if ms < 0:
            ctx.raise_last("time_read")
        emit(what=f"read-only stream, {name}", bytes=b16, regions=n_buf, us_per_launch=round(ms * 1e3, 2),
             GB_per_s=round(b16 / ms / 1e6, 1), frac_of_8TB=round(b16 / ms / 1e6 / 8000, 3))
    buf.free()
    ctx.close()


def config1(ctx, nbuf=48, iters=96):
    rows = cols = 4096
    bufs = [ctx.synth_quant(S.Q4_K, rows, cols, 1000 + i) for i in range(nbuf)]
    x = ctx.synth_normal(cols, 5)
    y = ctx.alloc(4 * rows * nbuf)
    arr = (C.c_void_p * nbuf)(*[b.ptr for b in bufs])
    H.lib.gq_hip_time_matvec(ctx.h, S.Q4_K, arr, nbuf, rows, cols, x.ptr, y.ptr, 8)
    ms = H.lib.gq_hip_time_matvec(ctx.h, S.Q4_K, arr, nbuf, rows, cols, x.ptr, y.ptr, iters)
    alg = S.qbytes(S.Q4_K, rows, cols) + 4 * rows + 4 * cols
    emit(config=1, what="Q4_K matvec 4096x4096, 48 rotating matrices", us_per_launch=round(ms * 1e3, 2),
         algorithmic_bytes=alg, GB_per_s=round(alg / ms / 1e6, 1))
    for b in bufs:
        b.free()
    x.free(), y.free()


def config2(ctx):
    spec, pre, n = S.TINYLLAMA, 512, 128
    dm = H.DeviceModel(ctx, spec, 640, prefill=pre)
    ctx.sync()
    dm.decode_loop(1, pre, 8, use_graph=True)
    ctx.sync()
    t0 = time.perf_counter()
    toks, dev_ms = dm.decode_loop(1, pre, n, use_graph=True)
    ctx.sync()
    wall = time.perf_counter() - t0
    emit(config=2, what="TinyLlama-shape greedy decode, 128 steps from pos 512 (graph replay)",
         tok_per_s=round(n / wall, 1), ref_definition_tok_per_s=round((n - 1) / wall, 1),
         ms_per_token=round(wall * 1e3 / n, 4), weight_bytes_per_token=spec.weight_bytes_per_token(),
         first_tokens=[int(t) for t in toks[:8]])


def config4(ctx):
    spec = S.LLAMA8B
    top = 32768
    dm = H.DeviceModel(ctx, spec, top + 64, prefill=top)
    ctx.sync()
    q = ctx.synth_normal(spec.n_heads * spec.head_dim, 3)
    out = ctx.alloc(4 * spec.n_heads * spec.head_dim)
    for L in (8192, 16384, 32768):
        H.lib.gq_hip_time_attention(ctx.h, 0, L - 1, q.ptr, out.ptr, 8)
        ms = H.lib.gq_hip_time_attention(ctx.h, 0, L - 1, q.ptr, out.ptr, 64)
        alg = 2 * spec.n_kv_heads * L * spec.head_dim * 4
        emit(config=4, what=f"split-K GQA attention per layer, {L} positions (partial + merge)",
             us_per_layer=round(ms * 1e3, 2), kv_bytes=alg, GB_per_s=round(alg / ms / 1e6, 1))
    q.free(), out.free()


def config4_restore():
    ctx = H.Context(0)
    L, nkv, hd, ms_ = 32, 8, 128, 4096
    ctx.kv_init(L, nkv, hd, ms_, 500000.0)
    ctx.kv_prefill_synth(11, 12, ms_)
    before = [ctx.kv_read_layer(l) for l in (0, L - 1)]
    fd, path = tempfile.mkstemp(suffix=".lctx")
    os.close(fd)
    try:
        ctx.check(ctx.lctx_save(path, ms_), "lctx_save")
        size = os.path.getsize(path)
        img = H.lib.gq_hip_host_alloc_pinned(size)
        if not img:
            raise H.HipError("pinned allocation failed")
        with open(path, "rb") as f:
            f.readinto((C.c_char * size).from_address(img))
        ctx.kv_prefill_synth(99, 98, ms_)  # overwrite the cache before restoring
        times = []
        for _ in range(3):
            rc, pos, ms = ctx.lctx_restore_image(img, size)
            ctx.check(rc, "lctx_restore_image")
            times.append(ms)
        after = [ctx.kv_read_layer(l) for l in (0, L - 1)]
        exact = all(np.array_equal(a[i].view(np.uint32), b[i].view(np.uint32))
                    for a, b in zip(before, after) for i in (0, 1))
        kv_bytes = 2 * L * nkv * ms_ * hd * 4
        best = min(times)
        emit(config=4, what=".lctx restore, 4096-token prefix (max_seq 4096) from pinned host memory",
             file_bytes=size, kv_bytes=kv_bytes, ms=round(best, 3), GB_per_s=round(kv_bytes / best / 1e6, 1),
             bit_exact_layers_0_and_31=exact, restored_pos=pos)
        H.lib.gq_hip_host_free_pinned(img)
    finally:
        os.unlink(path)
        ctx.close()


def config5(ctx, T=512, iters=20):
    spec = S.LLAMA8B
    H_, F = spec.hidden, spec.ff
    shapes = [("q/o", H_, H_), ("k/v", spec.n_kv_heads * spec.head_dim, H_), ("gate/up", F, H_), ("down", H_, F)]
    for dt, name in ((S.Q4_K, "Q4_K"), (S.Q6_K, "Q6_K")):
        for what, N, K in shapes:
            w = ctx.synth_quant(dt, N, K, 77 + N + K)
            x = ctx.synth_normal(T * K, 5)
            y = ctx.alloc(4 * T * N)

            # device time of the GEMM launches alone (x's bf16 copy and the
            # Q6_K unit-layout copy made before the timed region)
            ms = H.lib.gq_hip_time_prefill_gemm(ctx.h, dt, w.ptr, N, K, x.ptr, T, y.ptr, iters)
            if ms < 0:
                ctx.raise_last("time_prefill_gemm")
            dt_s = ms * 1e-3
            flop = 2.0 * T * N * K
            emit(config=5, what=f"prefill GEMM {name} {what}: {T} tokens x {N}x{K}", us_per_launch=round(dt_s * 1e6, 2),
                 gflop=round(flop / 1e9, 2), TFLOP_per_s=round(flop / dt_s / 1e12, 1),
                 weight_bytes=S.qbytes(dt, N, K))
            w.free(), x.free(), y.free()
    # gate and up in one launch with SwiGLU in the epilogue (the model's form)
    wg, wu = ctx.synth_quant(S.Q4_K, F, H_, 91), ctx.synth_quant(S.Q4_K, F, H_, 92)
    x = ctx.synth_normal(T * H_, 5)
    act = ctx.alloc(2 * T * F)

    def gu():
        ctx.check(H.lib.gq_hip_prefill_gate_up_dev(ctx.h, S.Q4_K, wg.ptr, wu.ptr, F, H_, x.ptr, T, act.ptr), "gate/up")
    gu()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(iters):
        gu()
    ctx.sync()
    dt_s = (time.perf_counter() - t0) / iters
    flop = 2 * 2.0 * T * F * H_
    emit(config=5, what=f"prefill gate+up+SwiGLU Q4_K: {T} tokens x 2x{F}x{H_} (incl. fp32->bf16 of x)",
         us_per_launch=round(dt_s * 1e6, 2), gflop=round(flop / 1e9, 2), TFLOP_per_s=round(flop / dt_s / 1e12, 1))
    for b in (wg, wu, x, act):
        b.free()
    # RoPE + append + causal attention of T tokens from position 0
    nh, nkv, hd = spec.n_heads, spec.n_kv_heads, spec.head_dim
    ctx.kv_init(1, nkv, hd, T + 128, spec.rope_theta)
    q, k, v = ctx.synth_normal(T * nh * hd, 1), ctx.synth_normal(T * nkv * hd, 2), ctx.synth_normal(T * nkv * hd, 3)
    o = ctx.alloc(4 * T * nh * hd)
    ctx.check(ctx.prefill_attention_dev(0, 0, T, nh, q, k, v, o), "prefill attention")
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(iters):
        ctx.check(ctx.prefill_attention_dev(0, 0, T, nh, q, k, v, o), "prefill attention")
    ctx.sync()
    dt_s = (time.perf_counter() - t0) / iters
    flop = 4.0 * nh * hd * T * (T + 1) / 2  # q.k and p.v over the causal triangle
    emit(config=5, what=f"RoPE + append + causal attention, {T} tokens, 32 heads / 8 KV heads, hd 128",
         us_per_layer=round(dt_s * 1e6, 2), gflop=round(flop / 1e9, 3), TFLOP_per_s=round(flop / dt_s / 1e12, 2))
    for b in (q, k, v, o):
        b.free()
    ctx.close()
    # forward() over a T-token prompt through the whole model
    ctx = H.Context(0)
    dm = H.DeviceModel(ctx, spec, T + 128)
    toks = np.random.default_rng(5).integers(0, spec.vocab, T).astype(np.int32)
    dm.prefill(toks, 0, want_logits=False)
    best = None
    for _ in range(3):
        t0 = time.perf_counter()
        nxt, _, _, dev_ms = dm.prefill(toks, 0, want_logits=False)
        wall = time.perf_counter() - t0
        best = wall if best is None else min(best, wall)
    emit(config=5, what=f"forward() of a {T}-token prompt, 8B shape, 32 layers (prefill)", ms=round(best * 1e3, 3),
         device_ms=round(dev_ms, 3), tok_per_s=round(T / best, 1), next_token=int(nxt))
    ctx.close()


def run_gemm(dtype, rows, cols, T, iters):
    ctx = H.Context(0)
    w = ctx.synth_quant(dtype, rows, cols, 7)
    x = ctx.synth_normal(T * cols, 5)
    y = ctx.alloc(4 * T * rows)
    t0 = None
    for i in range(iters + 1):
        if i == 1:
            ctx.sync()
            t0 = time.perf_counter()
        ctx.check(H.lib.gq_hip_prefill_gemm_dev(ctx.h, dtype, 0, w.ptr, rows, cols, x.ptr, T, y.ptr, None), "gemm")
    ctx.sync()
    dt = (time.perf_counter() - t0) / iters
    emit(what=f"prefill GEMM dtype {dtype} {T} x {rows}x{cols}", us_per_launch=round(dt * 1e6, 2),
         TFLOP_per_s=round(2.0 * T * rows * cols / dt / 1e12, 1))
    ctx.close()


def run_sample(vocab, iters):
    ctx = H.Context(0)
    x = (np.random.default_rng(5).standard_normal(vocab) * 3.0).astype(np.float32)
    xd = ctx.upload(x)
    for what, T, k, p in (("greedy", 0.0, 0, 1.0), ("top-k 40, T 0.8", 0.8, 40, 1.0),
                          ("top-p 0.9, T 0.8", 0.8, 0, 0.9), ("temperature 0.8", 0.8, 0, 1.0)):
        rnd = 12345
        for _ in range(3):
            ctx.check(min(0, H.lib.gq_hip_sample_dev(ctx.h, xd.ptr, vocab, T, k, p, rnd)), "sample")
        t0 = time.perf_counter()
        for i in range(iters):
            tok = H.lib.gq_hip_sample_dev(ctx.h, xd.ptr, vocab, T, k, p, rnd + i)
            ctx.check(min(0, tok), "sample")
        dt = (time.perf_counter() - t0) / iters
        emit(what=f"on-device sampling, {what}", vocab=vocab, us_per_call=round(dt * 1e6, 1),
             logits_bytes_not_copied=4 * vocab)
    ctx.close()


def run_configs():
    ctx = H.Context(0)
    config1(ctx)
    ctx.close()
    ctx = H.Context(0)
    config2(ctx)
    ctx.close()
    ctx = H.Context(0)
    config4(ctx)
    ctx.close()
    config4_restore()


def run_upload():
    """Weight upload of the 8B shape's per-layer tensors (4.6 GB in all) from
    pageable host memory through gq_hip_upload_weight (pinned staging),
    tensor by tensor as the loader uploads them: GB/s over the whole model,
    and hipMemGetInfo before the context, with the weights resident, and
    after gq_hip_destroy."""
    spec = S.LLAMA8B
    sizes = []
    for l in range(spec.n_layers):
        for k, dt in spec.dtypes(l).items():
            sizes.append(S.qbytes(dt, *spec.shape(k)))
    sizes.append(S.qbytes(spec.lm_head_dtype, *spec.shape("lm_head")))
    sizes.append(S.qbytes(spec.embed_dtype, *spec.shape("embed")))
    host = np.random.default_rng(0).integers(0, 256, max(sizes), dtype=np.uint8)
    warm = H.Context(0)
    H.lib.gq_hip_upload_weight(warm.h, host.ctypes.data, 1 << 20)
    warm.close()
    free0, total = H.mem_info(0)
    ctx = H.Context(0)
    t0 = time.perf_counter()
    for n in sizes:
        if not H.lib.gq_hip_upload_weight(ctx.h, host.ctypes.data, n):
            ctx.raise_last("upload")
    dt = time.perf_counter() - t0
    free1, _ = H.mem_info(0)
    ctx.close()
    free2, _ = H.mem_info(0)
    tot = sum(sizes)
    emit(what="weight upload, Llama-3.1-8B-shape Q4_K_M, tensor by tensor from pageable host memory "
              "(pinned double-buffered staging)", tensors=len(sizes), bytes=tot, seconds=round(dt, 3),
         GB_per_s=round(tot / dt / 1e9, 2), free_before=free0, free_resident=free1, free_after_destroy=free2,
         returned_all=free2 == free0, total=total)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("copy")
    c.add_argument("--mib", type=int, default=256)
    c.add_argument("--iters", type=int, default=20)
    sub.add_parser("configs")
    smp = sub.add_parser("sample")
    smp.add_argument("--vocab", type=int, default=128256)
    smp.add_argument("--iters", type=int, default=50)
    sub.add_parser("config5")
    sub.add_parser("upload")
    fl = sub.add_parser("floor")
    fl.add_argument("--iters", type=int, default=64)
    g = sub.add_parser("gemm")
    g.add_argument("--dtype", type=int, default=S.Q4_K)
    g.add_argument("--rows", type=int, default=4096)
    g.add_argument("--cols", type=int, default=4096)
    g.add_argument("--tokens", type=int, default=512)
    g.add_argument("--iters", type=int, default=20)
    a = ap.parse_args()
    if a.cmd == "copy":
        run_copy(a.mib, a.iters)
    elif a.cmd == "configs":
        run_configs()
    elif a.cmd == "sample":
        run_sample(a.vocab, a.iters)
    elif a.cmd == "config5":
        config5(H.Context(0))
    elif a.cmd == "upload":
        run_upload()
    elif a.cmd == "floor":
        run_floor(a.iters)
    elif a.cmd == "gemm":
        run_gemm(a.dtype, a.rows, a.cols, a.tokens, a.iters)


if __name__ == "__main__":
    main()
