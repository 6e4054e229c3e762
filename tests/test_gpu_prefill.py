"""The prefill chunk (config 5) on the GPU.

GEMM, Y = X W^T for T tokens on the bf16 matrix cores; two references on the
same seeded inputs:

* exact-input reference: X and the dequantized weights rounded to bf16 the
  way the kernel rounds them (Q4_K: w = d sc q - dmin m rounded once to fp32;
  Q6_K: w = (d sc) q, exact in fp32; then bf16 nearest-even), products and
  sums in fp64.  Only the kernel's fp32 accumulation order differs:
  tolerance 1e-5 relative L2.  This pins indexing, operand layouts and the
  block decodes.
* full-precision reference: fp64 GEMM of the fp32 X and the exactly
  dequantized weights (what the reference's T sequential fp32 matvecs
  approximate, engine.c:119-152).  bf16 inputs cost ~2^-9 relative per
  product: tolerance 1e-2 relative L2 (observed ~3e-3).

RoPE + append + causal attention of T tokens (the fp32-MFMA flash kernel):
the cache rows bit-exact with the oracle's RoPE, each token's attention
within 1e-5 of the oracle and of the decode kernel at its position.

Whole-model prefill (forward() over a prompt, engine.c:559-595) against T
sequential oracle steps (bit-exact with the reference's forward()): the
projections see bf16 inputs, so the last token's logits and the new cache
rows are held to 3e-2 relative L2 (observed about 5e-3) and the next greedy
token must agree."""
import numpy as np
import pytest

from guanaco_amd import spec as S
from util import bits, dequant_q4k_f64, dequant_q6k_f64, dequant_q8_0_f64, rel_l2

pytestmark = pytest.mark.gpu


def bf16_round(a):
    b = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return b.astype(np.uint32).view(np.float32)


def q4k_dequant_kernel_order(w, rows, cols):
    """Per weight: fp32(d*sc*q - dmin*m) with one rounding (the kernel's
    fma), d*sc and dmin*m exact in fp32."""
    blk = w.reshape(rows, cols // 256, 144)
    d = blk[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dm = blk[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    sc = blk[:, :, 4:16].astype(np.int64)
    qs = blk[:, :, 16:144].astype(np.int64)
    out = np.empty((rows, cols // 256, 256), np.float64)
    for j in range(8):
        if j < 4:
            s, m = sc[..., j] & 63, sc[..., j + 4] & 63
        else:
            s = (sc[..., j + 4] & 15) | ((sc[..., j - 4] >> 6) << 4)
            m = (sc[..., j + 4] >> 4) | ((sc[..., j] >> 6) << 4)
        chunk = qs[..., 32 * (j // 2):32 * (j // 2) + 32]
        q = (chunk >> 4) if (j & 1) else (chunk & 15)
        a = (d * s).astype(np.float32).astype(np.float64)
        mm = (dm * m).astype(np.float32).astype(np.float64)
        out[..., 32 * j:32 * j + 32] = (a[..., None] * q - mm[..., None]).astype(np.float32)
    return out.reshape(rows, cols)


SHAPES = [(64, 128, 256), (100, 256, 512), (512, 1024, 4096), (130, 384, 1024)]


@pytest.mark.parametrize("T,N,K", SHAPES)
@pytest.mark.parametrize("mode", [0, 1])
def test_prefill_gemm(ctx, orc, T, N, K, mode):
    _gemm_case(ctx, orc, S.Q4_K, T, N, K, mode)


@pytest.mark.parametrize("T,N,K", [(64, 128, 512), (100, 256, 512), (512, 1024, 4096), (77, 384, 1536),
                                   (33, 128, 3584)])
@pytest.mark.parametrize("mode", [0, 1])
def test_prefill_gemm_q6k(ctx, orc, T, N, K, mode):
    _gemm_case(ctx, orc, S.Q6_K, T, N, K, mode)


@pytest.mark.parametrize("T,N,K", [(64, 128, 256), (100, 256, 512), (512, 1024, 4096), (77, 384, 1536),
                                   (33, 128, 5632), (512, 2048, 2048)])
@pytest.mark.parametrize("mode", [0, 1])
def test_prefill_gemm_q8_0(ctx, orc, T, N, K, mode):
    """Q8_0 weights (quant_matvec_q8_0.c:5-10): w = d q is exact in fp32, so
    the exact-input reference is bf16(d q) against bf16(x)."""
    _gemm_case(ctx, orc, S.Q8_0, T, N, K, mode)


def _dequant(dtype, w, rows, cols):
    return {S.Q4_K: dequant_q4k_f64, S.Q6_K: dequant_q6k_f64, S.Q8_0: dequant_q8_0_f64}[dtype](w, rows, cols)


def _kernel_weights(dtype, w, rows, cols):
    """The fp32 weights the kernel rounds to bf16: Q4_K in its fma order,
    Q6_K and Q8_0 exact."""
    if dtype == S.Q4_K:
        return q4k_dequant_kernel_order(w, rows, cols)
    return _dequant(dtype, w, rows, cols).astype(np.float32)


def _gemm_case(ctx, orc, dtype, T, N, K, mode):
    import guanaco_amd.hip as H
    seed = (T << 20) ^ (N << 8) ^ K ^ (dtype << 28)
    w = orc.synth_quant(dtype, seed, N, K)
    x = orc.synth_normal(seed + 1, T * K).reshape(T, K)
    r = orc.synth_normal(seed + 2, T * N).reshape(T, N)
    wd, xd = ctx.upload_weight(w), ctx.upload(x)
    yd = ctx.upload(r) if mode == 1 else ctx.alloc(4 * T * N)
    rc = H.lib.gq_hip_prefill_gemm_dev(ctx.h, dtype, mode, wd, N, K, xd.ptr, T, yd.ptr,
                                       yd.ptr if mode == 1 else None)
    assert rc == 0
    y = yd.download(count=T * N).reshape(T, N)
    base = r.astype(np.float64) if mode == 1 else 0.0
    wf = _dequant(dtype, w, N, K)
    wk = _kernel_weights(dtype, w, N, K)
    exact_in = bf16_round(x).astype(np.float64) @ bf16_round(wk).astype(np.float64).T
    assert rel_l2(y, base + exact_in) < 1e-5
    full = x.astype(np.float64) @ wf.T
    e = rel_l2(y - base, full)
    assert e < 1e-2, e
    H.lib.gq_hip_free(ctx.h, wd)
    xd.free(), yd.free()


@pytest.mark.parametrize("dtype,N,K,mode", [
    (S.Q4_K, 4096, 4096, 0),    # q / o
    (S.Q4_K, 14336, 4096, 0),   # gate / up
    (S.Q4_K, 4096, 14336, 1),   # down + residual
    (S.Q6_K, 4096, 14336, 1),   # the Q6_K down of the Q4_K_M mix
    (S.Q6_K, 14336, 4096, 0),   # Q6_K gate / up: 128-token tiles from the unit layout
])
def test_prefill_gemm_config5_shapes(ctx, orc, dtype, N, K, mode):
    """Config 5's full 512-token GEMMs on the 8B projection shapes; every
    token is checked on 384 sampled output rows (first and last included)
    against the exact-input fp64 reference (1e-5) and the full-precision one
    (1e-2)."""
    import guanaco_amd.hip as H
    T = 512
    seed = 0xC0F5 ^ (N << 8) ^ K ^ (dtype << 28)
    print(f"prefill GEMM {T}x{N}x{K} dtype {dtype} mode {mode}", flush=True)
    w = orc.synth_quant(dtype, seed, N, K)
    x = orc.synth_normal(seed + 1, T * K).reshape(T, K)
    r = orc.synth_normal(seed + 2, T * N).reshape(T, N)
    wd, xd = ctx.upload_weight(w), ctx.upload(x)
    yd = ctx.upload(r) if mode == 1 else ctx.alloc(4 * T * N)
    assert H.lib.gq_hip_prefill_gemm_dev(ctx.h, dtype, mode, wd, N, K, xd.ptr, T, yd.ptr,
                                         yd.ptr if mode == 1 else None) == 0
    y = yd.download(count=T * N).reshape(T, N)
    H.lib.gq_hip_free(ctx.h, wd)
    xd.free(), yd.free()
    idx = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(seed).choice(N, 382, replace=False)]))
    ws = np.ascontiguousarray(w.reshape(N, -1)[idx]).reshape(-1)
    n = idx.size
    wf = dequant_q4k_f64(ws, n, K) if dtype == S.Q4_K else dequant_q6k_f64(ws, n, K)
    wk = q4k_dequant_kernel_order(ws, n, K) if dtype == S.Q4_K else wf.astype(np.float32)
    base = r[:, idx].astype(np.float64) if mode == 1 else 0.0
    ys = y[:, idx]
    exact_in = bf16_round(x).astype(np.float64) @ bf16_round(wk).astype(np.float64).T
    assert rel_l2(ys, base + exact_in) < 1e-5
    assert rel_l2(ys - base, x.astype(np.float64) @ wf.T) < 1e-2


def test_prefill_gemm_rejects_bad_shapes(ctx):
    import guanaco_amd.hip as H
    buf = ctx.alloc(1 << 20)
    assert H.lib.gq_hip_prefill_gemm_dev(ctx.h, S.Q4_K, 0, buf.ptr, 100, 256, buf.ptr, 4, buf.ptr, None) != 0
    assert H.lib.gq_hip_prefill_gemm_dev(ctx.h, S.Q4_K, 0, buf.ptr, 128, 300, buf.ptr, 4, buf.ptr, None) != 0
    assert H.lib.gq_hip_prefill_gemm_dev(ctx.h, S.F32, 0, buf.ptr, 128, 256, buf.ptr, 4, buf.ptr, None) != 0
    assert H.lib.gq_hip_prefill_gemm_dev(ctx.h, S.Q8_0, 0, buf.ptr, 128, 288, buf.ptr, 4, buf.ptr, None) != 0
    assert H.lib.gq_hip_prefill_gemm_dev(ctx.h, S.Q6_K, 0, buf.ptr, 128, 256, buf.ptr, 4, buf.ptr, None) == -2
    buf.free()


def silu_mul_f32(g, u):
    g = g.astype(np.float32)
    with np.errstate(over="ignore"):
        sig = np.float32(1) / (np.float32(1) + np.exp(np.float32(0) - g))
    return (g * sig) * u.astype(np.float32)


@pytest.mark.parametrize("dtype,T,N,K", [(S.Q4_K, 512, 1024, 4096), (S.Q4_K, 70, 192, 512),
                                         (S.Q6_K, 100, 256, 1024), (S.Q6_K, 100, 256, 4096),
                                         (S.Q8_0, 100, 256, 1024), (S.Q8_0, 512, 1024, 2048)])
def test_prefill_gate_up_swiglu(ctx, orc, dtype, T, N, K):
    """gate and up in one launch with SiLU(gate) * up in the epilogue
    (kernels_cpu.c:312-389), bf16 out: against the exact-input reference
    (bf16 operands, fp64 sums, the SwiGLU in fp32 and bf16 rounding as the
    kernel does; only the accumulation order differs) and against fp64."""
    import guanaco_amd.hip as H
    seed = (T << 16) ^ (N << 4) ^ K
    wg, wu = orc.synth_quant(dtype, seed, N, K), orc.synth_quant(dtype, seed + 1, N, K)
    x = orc.synth_normal(seed + 2, T * K).reshape(T, K)
    gd, ud, xd = ctx.upload_weight(wg), ctx.upload_weight(wu), ctx.upload(x)
    act = ctx.alloc(2 * T * N)
    assert H.lib.gq_hip_prefill_gate_up_dev(ctx.h, dtype, gd, ud, N, K, xd.ptr, T, act.ptr) == 0
    a16 = act.download(np.uint16, count=T * N).reshape(T, N)
    got = (a16.astype(np.uint32) << 16).view(np.float32)
    deq = lambda w, n, k: _dequant(dtype, w, n, k)  # noqa: E731
    kern = lambda w: _kernel_weights(dtype, w, N, K)  # noqa: E731
    xb = bf16_round(x).astype(np.float64)
    g = xb @ bf16_round(kern(wg)).astype(np.float64).T
    u = xb @ bf16_round(kern(wu)).astype(np.float64).T
    assert rel_l2(got, bf16_round(silu_mul_f32(g, u))) < 1e-3
    g64, u64 = x.astype(np.float64) @ deq(wg, N, K).T, x.astype(np.float64) @ deq(wu, N, K).T
    with np.errstate(over="ignore"):
        assert rel_l2(got, g64 / (1 + np.exp(-g64)) * u64) < 2e-2
    act.free(), xd.free()
    H.lib.gq_hip_free(ctx.h, gd), H.lib.gq_hip_free(ctx.h, ud)


@pytest.mark.parametrize("T,N,K", [(512, 14336, 4096), (300, 11008, 2048), (257, 11008, 1024)])
def test_prefill_gate_up_wide_tile(ctx, orc, T, N, K):
    """The fused Q4_K gate/up launch on the wide tile (64 rows per wave),
    which the launcher takes when the 128-row tiles alone fill the GPU
    (config 5's 2 x 14336 x 4096; ragged 300- and 257-token cases, the
    last with one token in its last tile).  Rows are
    independent, so each half of the rows runs again as a launch of its own,
    which on 256 CUs takes the 32-row tile without a K split (7168 rows at
    512 tokens, 5504 at 300 and 257): the same sums in the same order, so the halves
    must agree bit for bit with the wide launch.  Sampled rows are held to
    the exact-input reference as test_prefill_gate_up_swiglu does."""
    import guanaco_amd.hip as H
    seed = 0x5EED ^ (T << 16) ^ N
    print(f"prefill gate/up wide tile {T}x{N}x{K}", flush=True)
    wg, wu = orc.synth_quant(S.Q4_K, seed, N, K), orc.synth_quant(S.Q4_K, seed + 1, N, K)
    x = orc.synth_normal(seed + 2, T * K).reshape(T, K)
    gd, ud, xd = ctx.upload_weight(wg), ctx.upload_weight(wu), ctx.upload(x)
    half = N // 2
    act, sub = ctx.alloc(2 * T * N), ctx.alloc(2 * T * half)
    assert H.lib.gq_hip_prefill_gate_up_dev(ctx.h, S.Q4_K, gd, ud, N, K, xd.ptr, T, act.ptr) == 0
    wide = act.download(np.uint16, count=T * N).reshape(T, N)
    if ctx.info()[0] == 256:
        rowbytes = K // 256 * 144
        for r0 in (0, half):
            assert H.lib.gq_hip_prefill_gate_up_dev(ctx.h, S.Q4_K, gd + r0 * rowbytes, ud + r0 * rowbytes, half, K,
                                                    xd.ptr, T, sub.ptr) == 0
            narrow = sub.download(np.uint16, count=T * half).reshape(T, half)
            assert np.array_equal(wide[:, r0:r0 + half], narrow), r0
    idx = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(seed).choice(N, 254, replace=False)]))
    n = idx.size
    pick = lambda w: np.ascontiguousarray(w.reshape(N, -1)[idx]).reshape(-1)  # noqa: E731
    xb = bf16_round(x).astype(np.float64)
    g = xb @ bf16_round(q4k_dequant_kernel_order(pick(wg), n, K)).astype(np.float64).T
    u = xb @ bf16_round(q4k_dequant_kernel_order(pick(wu), n, K)).astype(np.float64).T
    got = (wide[:, idx].astype(np.uint32) << 16).view(np.float32)
    assert rel_l2(got, bf16_round(silu_mul_f32(g, u))) < 1e-3
    act.free(), sub.free(), xd.free()
    H.lib.gq_hip_free(ctx.h, gd), H.lib.gq_hip_free(ctx.h, ud)


@pytest.mark.parametrize("nh,nkv,hd,pre,T,ms", [
    (32, 8, 128, 0, 512, 640),     # config 5: a 512-token chunk from position 0
    (32, 8, 128, 300, 200, 640),   # after a cached prefix
    (32, 4, 64, 5, 130, 135),      # TinyLlama shape, ends at the cache end (max_seq % 16 != 0)
    (8, 8, 64, 0, 3, 16),          # G = 1, three tokens
    (64, 8, 128, 7, 33, 64),       # G = 8, two tokens per tile
    (16, 8, 64, 1, 21, 40),        # G = 2
])
def test_prefill_attention(ctx, orc, nh, nkv, hd, pre, T, ms):
    from oracle import HostKV, fptr
    theta = 500000.0
    ctx.kv_init(1, nkv, hd, ms, theta)
    seed_k, seed_v = 0x5EED + pre, 0xFEED + T
    if pre:
        ctx.kv_prefill_synth(seed_k, seed_v, pre)
    rng = np.random.default_rng(T * 1000 + pre)
    q = rng.standard_normal((T, nh * hd)).astype(np.float32)
    k = rng.standard_normal((T, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((T, nkv * hd)).astype(np.float32)
    qb, kb, vb, ob = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.alloc(4 * T * nh * hd)
    assert ctx.prefill_attention_dev(0, pre, T, nh, qb, kb, vb, ob) == 0
    out = ob.download(count=T * nh * hd).reshape(T, nh * hd)
    qr = qb.download(count=T * nh * hd).reshape(T, nh * hd)
    # RoPE and the appended rows bit-exact with the oracle
    kv = HostKV(1, nkv, hd, ms)
    for arr, seed in ((kv.k, seed_k), (kv.v, seed_v)):
        orc.lib.orc_synth_kv(seed, fptr(arr), 1, nkv, hd, ms, pre)
    kr = np.empty_like(k)
    for t in range(T):
        q2, k2 = orc.rope(q[t], k[t], nh, nkv, hd, pre + t, theta)
        assert np.array_equal(bits(qr[t]), bits(q2)), t
        kr[t] = k2
    kvk, kvv = kv.k.reshape(nkv, ms, hd), kv.v.reshape(nkv, ms, hd)
    kvk[:, pre:pre + T] = kr.reshape(T, nkv, hd).transpose(1, 0, 2)
    kvv[:, pre:pre + T] = v.reshape(T, nkv, hd).transpose(1, 0, 2)
    dk, dv = ctx.kv_read_layer(0)
    assert np.array_equal(bits(dk), bits(kv.k)) and np.array_equal(bits(dv), bits(kv.v))
    # each token against the oracle (fp32 throughout, only the summation
    # order differs) and against the decode kernel at its position
    q1, o1 = ctx.alloc(4 * nh * hd), ctx.alloc(4 * nh * hd)
    for t in sorted({0, 1, 2, 15, 16, 17, T // 2, T - 2, T - 1} & set(range(T))):
        ref = orc.attention(qr[t], kv, 0, nh, pre + t)
        assert rel_l2(out[t], ref) < 1e-5, t
        if nh // nkv in (1, 4, 8):  # the decode kernel's group sizes
            q1.upload(qr[t])
            assert ctx.attention_dev(0, pre + t, nh, q1, o1) == 0
            assert rel_l2(out[t], o1.download()) < 1e-5, t
    for b in (qb, kb, vb, ob, q1, o1):
        b.free()


def test_prefill_attention_rejects_bad_positions(ctx):
    ctx.kv_init(1, 2, 64, 32, 500000.0)
    b = ctx.alloc(4 * 40 * 8 * 64)
    assert ctx.prefill_attention_dev(0, 30, 3, 8, b, b, b, b) == -5
    assert ctx.prefill_attention_dev(0, -1, 3, 8, b, b, b, b) == -5
    assert ctx.prefill_attention_dev(0, 0, 0, 8, b, b, b, b) == -1
    assert ctx.prefill_attention_dev(0, 0, 3, 7, b, b, b, b) == -1
    b.free()


PF_TOL = 3e-2


@pytest.mark.parametrize("pre,T,ms", [(0, 48, 64), (24, 39, 64), (0, 600, 640)])
def test_prefill_model_vs_oracle(ctx, orc, pre, T, ms):
    """forward() over a T-token prompt at pos `pre` (the reference's own
    prefill call, generate.c:200-226), then one decode step from it."""
    import guanaco_amd.hip as H
    from oracle import HostModel
    from guanaco_amd.synth import tensor_seed
    spec = S.TINY_TEST
    hm = HostModel(orc, spec, ms)
    dm = H.DeviceModel(ctx, spec, ms, prefill=pre)
    kv = hm.new_kv()
    if pre:
        kv.prefill(orc, spec, pre)
    rng = np.random.default_rng(T + pre)
    toks = rng.integers(0, spec.vocab, T).astype(np.int32)
    nxt, lg, hid, ms_dev = dm.prefill(toks, pre, want_hidden=True)
    for t in range(T):
        t_cpu, lc, _ = hm.forward(kv, int(toks[t]), pre + t)
    assert rel_l2(lg, lc) < PF_TOL
    assert nxt == t_cpu
    for l in range(spec.n_layers):
        dk, dv = ctx.kv_read_layer(l)
        for d, h in ((dk, kv.view("k")[l]), (dv, kv.view("v")[l])):
            d = d.reshape(h.shape)
            assert np.array_equal(d[:, :pre], h[:, :pre])          # the cached prefix untouched
            assert rel_l2(d[:, pre:pre + T], h[:, pre:pre + T]) < PF_TOL
    # decode continues from the prefilled cache
    t_gpu, lg2, _ = dm.forward(nxt, pre + T)
    t_cpu2, lc2, _ = hm.forward(kv, t_cpu, pre + T)
    assert rel_l2(lg2, lc2) < PF_TOL and t_gpu == t_cpu2
    print(f"prefill T={T} pre={pre}: logits rel {rel_l2(lg, lc):.2e}, device {ms_dev:.3f} ms")


@pytest.mark.parametrize("T,N,K,mode", [(96, 256, 4096, 0), (77, 384, 2048, 1), (512, 4096, 14336, 1)])
def test_prefill_q6k_unit_layout_vs_reference_layout(ctx, orc, T, N, K, mode):
    """Q6_K weights whose rows fall on 16-byte boundaries (K % 2048 == 0) go
    through the GEMM in the decode matvec's unit layout (a copy made per call
    here; a bound model reads the copy model bind made for the decode step):
    the same bf16 weights as the reference layout, which matvec path 3
    reads, summed in another K order.  The two agree to the accumulation
    order (1e-5, as against the exact-input reference) and are not the same
    bits, so the unit layout was read."""
    import guanaco_amd.hip as H
    seed = 0x5E9 ^ (T << 16) ^ (N << 4) ^ K
    w = orc.synth_quant(S.Q6_K, seed, N, K)
    x = orc.synth_normal(seed + 1, T * K).reshape(T, K)
    r = orc.synth_normal(seed + 2, T * N).reshape(T, N)
    wd, xd = ctx.upload_weight(w), ctx.upload(x)
    out = {}
    for path in ("auto", "auto_q6k_ref"):
        yd = ctx.upload(r) if mode == 1 else ctx.alloc(4 * T * N)
        with H.matvec_path(path):
            assert H.lib.gq_hip_prefill_gemm_dev(ctx.h, S.Q6_K, mode, wd, N, K, xd.ptr, T, yd.ptr,
                                                 yd.ptr if mode == 1 else None) == 0
        out[path] = yd.download(count=T * N)
        yd.free()
    assert np.abs(out["auto"]).sum() > 0
    assert rel_l2(out["auto"], out["auto_q6k_ref"]) < 1e-5
    assert not np.array_equal(bits(out["auto"]), bits(out["auto_q6k_ref"]))
    H.lib.gq_hip_free(ctx.h, wd)
    xd.free()


def test_prefill_q6k_unit_layout_model(orc):
    """A model whose Q6_K projections (v, o, down) have K % 2048 == 0 prefills
    from the unit-layout copies made at model bind (the down projection's is
    the decode step's own): logits and the last hidden state within 2e-3 of
    the reference layout's (matvec path 3; the K order of the sums differs,
    and the bf16 activations may round apart), and the prompt against the
    oracle as for the other models, on both."""
    import guanaco_amd.hip as H
    from oracle import HostModel
    spec = S.ModelSpec("q6k-steps-test", n_layers=2, hidden=2048, ff=4096, n_heads=16, n_kv_heads=4, vocab=1000,
                       layer_dtypes=dict(wv=S.Q6_K, wo=S.Q6_K, wd=S.Q6_K))
    c = H.Context(0)
    try:
        hm = HostModel(orc, spec, 64)
        dm = H.DeviceModel(c, spec, 64)
        toks = np.random.default_rng(7).integers(0, spec.vocab, 40).astype(np.int32)
        res = {}
        for path in ("auto", "auto_q6k_ref"):
            with H.matvec_path(path):
                res[path] = dm.prefill(toks, 0, want_hidden=True)
        (nxt, lg, hg, _), (nxt2, lg2, hg2, _) = res["auto"], res["auto_q6k_ref"]
        assert rel_l2(lg, lg2) < 2e-3 and rel_l2(hg, hg2) < 2e-3
        kv = hm.new_kv()
        for t in range(len(toks)):
            t_cpu, lc, _ = hm.forward(kv, int(toks[t]), t)
        assert rel_l2(lg, lc) < PF_TOL and rel_l2(lg2, lc) < PF_TOL and nxt == t_cpu and nxt2 == t_cpu
        print(f"unit layout vs reference layout: logits {rel_l2(lg, lg2):.2e}, hidden {rel_l2(hg, hg2):.2e}")
    finally:
        c.close()


def test_prefill_q8_0_model(orc):
    """A model with every weight Q8_0 prefills through the GEMM (the
    reference's prefill takes Q8_0 through linear_dispatch,
    engine.c:119-152): last-token logits and the new cache rows against T
    sequential oracle steps (PF_TOL), the next greedy token equal, and the
    result not the token-by-token one (prefill mode 1), which is held to
    the decode tolerance."""
    import guanaco_amd.hip as H
    from oracle import HostModel
    spec = S.ModelSpec("tiny-q8_0", n_layers=2, hidden=512, ff=1024, n_heads=8, n_kv_heads=2, vocab=1000,
                       layer_dtypes={k: S.Q8_0 for k in S.LAYER_WEIGHTS}, embed_dtype=S.Q8_0,
                       lm_head_dtype=S.Q8_0)
    c = H.Context(0)
    try:
        hm = HostModel(orc, spec, 64)
        dm = H.DeviceModel(c, spec, 64)
        toks = np.random.default_rng(8).integers(0, spec.vocab, 48).astype(np.int32)
        kv = hm.new_kv()
        for t in range(len(toks)):
            t_cpu, lc, _ = hm.forward(kv, int(toks[t]), t)
        nxt, lg, _, _ = dm.prefill(toks, 0)
        assert rel_l2(lg, lc) < PF_TOL and nxt == t_cpu
        for l in range(spec.n_layers):
            dk, dv = c.kv_read_layer(l)
            for d, h in ((dk, kv.view("k")[l]), (dv, kv.view("v")[l])):
                d = d.reshape(h.shape)
                assert rel_l2(d[:, :len(toks)], h[:, :len(toks)]) < PF_TOL
        assert H.lib.gq_hip_set_prefill_mode(c.h, 1) == 0
        nxt1, lg1, _, _ = dm.prefill(toks, 0)
        assert rel_l2(lg1, lc) < 1e-3 and nxt1 == t_cpu
        assert not np.array_equal(bits(lg), bits(lg1))  # the GEMM path ran in mode 0
        print(f"Q8_0 model prefill: GEMM {rel_l2(lg, lc):.2e}, token by token {rel_l2(lg1, lc):.2e}")
    finally:
        c.close()


def test_prefill_after_rebinding_larger_models(orc):
    """One context binds a small model and prefills, then binds models with
    a wider FFN and a wider hidden size and prefills again: the prefill
    workspace is sized for the model bound last (it had kept the first
    model's sizes), each prompt against the oracle."""
    import guanaco_amd.hip as H
    from oracle import HostModel
    wide_h = S.ModelSpec("tiny-wide-hidden", n_layers=2, hidden=1024, ff=2048, n_heads=16, n_kv_heads=4,
                         vocab=1000, layer_dtypes=S._q6k_on_even)
    c = H.Context(0)
    try:
        for spec in (S.TINY_TEST, S.WIDE_FF_TEST, wide_h, S.TINY_TEST):
            print(f"prefill on a rebound context: {spec.name}", flush=True)
            hm = HostModel(orc, spec, 64)
            dm = H.DeviceModel(c, spec, 64)
            toks = np.random.default_rng(spec.hidden + spec.ff).integers(0, spec.vocab, 40).astype(np.int32)
            nxt, lg, _, _ = dm.prefill(toks, 0)
            kv = hm.new_kv()
            for t in range(len(toks)):
                t_cpu, lc, _ = hm.forward(kv, int(toks[t]), t)
            assert rel_l2(lg, lc) < PF_TOL and nxt == t_cpu, spec.name
    finally:
        c.close()


def test_prefill_token_by_token_fallback(ctx, orc):
    """A model whose Q6_K projections have cols % 512 != 0 (hidden 768) is
    not taken by the GEMM: the prefill runs the decode step per token, so
    it matches the decode path (and the oracle) to the decode tolerance."""
    import guanaco_amd.hip as H
    from oracle import HostModel
    spec = S.ModelSpec("tiny-fallback", n_layers=2, hidden=768, ff=1536, n_heads=12, n_kv_heads=3, vocab=1000,
                       layer_dtypes=S._q6k_on_even)
    hm = HostModel(orc, spec, 64)
    dm = H.DeviceModel(ctx, spec, 64)
    toks = np.random.default_rng(3).integers(0, spec.vocab, 20).astype(np.int32)
    nxt, lg, _, _ = dm.prefill(toks, 0)
    kv = hm.new_kv()
    for t in range(len(toks)):
        t_cpu, lc, _ = hm.forward(kv, int(toks[t]), t)
    assert rel_l2(lg, lc) < 1e-3 and nxt == t_cpu


def test_prefill_model_rejects_bad_input(ctx):
    import guanaco_amd.hip as H
    dm = H.DeviceModel(ctx, S.TINY_TEST, 64)
    with pytest.raises(H.HipError):
        dm.prefill(np.arange(10, dtype=np.int32), 60)      # past the cache
    with pytest.raises(H.HipError):
        dm.prefill(np.array([1, 2, 5000], np.int32), 0)    # token out of range
