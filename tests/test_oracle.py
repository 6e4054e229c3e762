"""Pins the CPU oracle (oracle/gq_oracle.c) before it is trusted as the parity
checker: the reference's own known-answer tests (tests/test_quant.c,
tests/test_kernels.c, tests/test_tokenizer.c), closed forms in float64,
exhaustive fp16 decoding, and bit-exact agreement with the reference's CPU
path compiled from its own sources (oracle/_ref, when built)."""
import numpy as np
import pytest

from oracle import F32, Q4_K, Q6_K, Q8_0, HostKV, HostModel, RefModel
from guanaco_amd import spec as S
from util import DEQUANT, bits, f16, q4k_block, rel_l2


def test_f16_exhaustive(orc):
    """Every binary16 encoding decodes exactly (quant_matvec_q4_k.c:18-45)."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([orc.lib.orc_f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(ref)[~nan])
    # NaN payload is kept (frac << 13), like the reference; the quiet bit is
    # not compared because ctypes returns the float through a Python double
    mask = 0x3FFFFF
    assert np.array_equal(bits(got)[nan] & mask, ((h[nan].astype(np.uint32) & 0x3FF) << 13) & mask)


def test_f32_to_f16_rne(orc):
    x = np.random.default_rng(1).standard_normal(20000).astype(np.float32) * np.float32(3.0)
    x = np.concatenate([x, np.float32([1e-7, 6e-8, 3e-8, 65504, 65520, 1e9, -0.0, 0.0, np.inf])])
    got = np.array([orc.lib.orc_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))


def test_q4k_kat_384(orc):
    """test_quant.c:94-139: d=1, dmin=0, scales 0x01, qs 0x12, x=1 -> 384."""
    blk = q4k_block(0x3C00, 0, np.full(12, 1, np.uint8), np.full(128, 0x12, np.uint8))
    y = orc.matvec(Q4_K, blk, 1, 256, np.ones(256, np.float32))
    assert abs(y[0] - 384.0) <= 1e-4


def test_q4k_scale_min_mapping(orc):
    """test_quant.c:141-218: crafted scale bytes exercise the 6-bit packing."""
    sc = np.array([0xC1, 0x42, 0x85, 0x0F, 0xF0, 0x3C, 0x83, 0x55, 0x12, 0x34, 0x56, 0x78], np.uint8)
    qs = np.zeros(128, np.uint8)
    qs[0], qs[32], qs[64], qs[96] = (2 << 4) | 1, (4 << 4) | 3, (6 << 4) | 5, (8 << 4) | 7
    blk = q4k_block(0x3C00, 0x3C00, sc, qs)
    x = np.zeros(256, np.float32)
    x[[0, 32, 64, 96, 128, 160, 192, 224]] = 1
    y = orc.matvec(Q4_K, blk, 1, 256, x)

    def su6(g):
        return sc[g] & 63 if g < 4 else (sc[g + 4] & 15) | ((sc[g - 4] >> 6) << 4)

    def mu6(g):
        return sc[g + 4] & 63 if g < 4 else (sc[g + 4] >> 4) | ((sc[g] >> 6) << 4)

    expect = sum(float(su6(g)) * (g + 1) - float(mu6(g)) for g in range(8))
    assert abs(y[0] - expect) <= 1e-4


def test_q8_0_kat(orc):
    """test_quant.c:26-68: scales 1.0 and 2.0, q = +/-(i+1), x = 1 -> -528."""
    blk = np.zeros(68, np.uint8)
    blk[0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    blk[2:34] = np.arange(1, 33, dtype=np.int8).view(np.uint8)
    blk[34:36] = np.frombuffer(np.uint16(0x4000).tobytes(), np.uint8)
    blk[36:68] = (-np.arange(1, 33)).astype(np.int8).view(np.uint8)
    y = orc.matvec(Q8_0, blk, 1, 64, np.ones(64, np.float32))
    assert abs(y[0] - (-528.0)) <= 1e-4


@pytest.mark.parametrize("dt,qk,bb", [(Q4_K, 256, 144), (Q6_K, 256, 210), (Q8_0, 32, 34)])
def test_matvec_error_codes(orc, dt, qk, bb):
    """-3 for a short byte_size, -2 for cols % block (quant_matvec_q4_k.c:143-158)."""
    w = np.zeros(bb * 4, np.uint8)
    x = np.zeros(4 * qk, np.float32)
    with pytest.raises(ValueError, match="rc=-3"):
        orc.matvec(dt, w, 1, 4 * qk, x, nbytes=bb * 4 - 1)
    with pytest.raises(ValueError, match="rc=-2"):
        orc.matvec(dt, w, 1, qk + 16, x)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K, Q8_0])
@pytest.mark.parametrize("rows,cols", [(1, 256), (8, 512), (33, 1024)])
def test_matvec_closed_form(orc, dt, rows, cols):
    """Against a float64 dequantise-then-dot written from the format alone."""
    w = orc.synth_quant(dt, 1000 + rows + dt, rows, cols)
    x = orc.synth_normal(7 + cols, cols)
    y = orc.matvec(dt, w, rows, cols, x)
    ref = DEQUANT[dt](w, rows, cols) @ x.astype(np.float64)
    assert rel_l2(y, ref) < 2e-6


@pytest.mark.parametrize("dt", [Q4_K, Q6_K, Q8_0])
@pytest.mark.parametrize("rows,cols", [(1, 256), (8, 512), (64, 1024), (37, 5632)])
def test_matvec_bitexact_vs_reference(orc, ref, dt, rows, cols):
    if dt == Q8_0:
        cols = cols // 8 * 8
    w = orc.synth_quant(dt, 77 + rows, rows, cols)
    x = orc.synth_normal(5 + cols, cols)
    assert np.array_equal(bits(orc.matvec(dt, w, rows, cols, x)), bits(ref.matvec(dt, w, rows, cols, x)))


def test_rmsnorm_properties(orc):
    """test_kernels.c:176-200: output RMS ~ 1 with unit weights."""
    x = np.random.default_rng(123).uniform(-5, 5, 64).astype(np.float32)
    out = orc.rmsnorm(x, np.ones(64, np.float32), 1e-6)
    assert abs(np.sqrt(np.mean(out.astype(np.float64) ** 2)) - 1.0) < 0.01
    x = np.random.default_rng(5).standard_normal(4096).astype(np.float32)
    w = np.random.default_rng(6).standard_normal(4096).astype(np.float32)
    r = 1 / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)
    assert rel_l2(orc.rmsnorm(x, w, 1e-6), w * (x * r)) < 1e-6


def test_softmax_properties(orc):
    """test_kernels.c:122-172: sums to 1, uniform, all -inf -> no NaN, single."""
    import ctypes as C
    from oracle import fptr

    def sm(v):
        a = np.array(v, np.float32)
        orc.lib.orc_softmax(fptr(a), a.size)
        return a

    assert abs(sm([1, 2, -0.5, 3, 0.1, -2, 4, 1.5]).sum() - 1) < 1e-6
    assert np.allclose(sm([5, 5, 5, 5]), 0.25, atol=1e-6)
    assert not np.isnan(sm([-np.inf] * 3)).any()
    assert abs(sm([42.0])[0] - 1.0) < 1e-6


def test_silu(orc):
    from oracle import fptr
    x = np.array([-2, -1, 0, 1, 2, 3, -3, 0.5, 7, -7], np.float32)
    ref = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    a = x.copy()
    orc.lib.orc_silu(fptr(a), a.size)
    assert np.abs(a - ref).max() < 1e-6


def test_greedy_first_max(orc):
    """tokenizer.c:175-185 and test_tokenizer.c:28-34: ties -> first index."""
    assert orc.argmax(np.array([1, 5, 2, 3], np.float32)) == 1
    assert orc.argmax(np.array([3, 1, 3, 2], np.float32)) == 0


def test_greedy_nan_vs_reference(orc, ref):
    """NaN logits: the oracle's scan picks what the compiled sample_greedy
    (tokenizer.c:175-185) picks — index 0 when logits[0] is NaN, and a NaN
    anywhere else skipped."""
    import ctypes as C
    ref.lib.sample_greedy.argtypes = [C.POINTER(C.c_float), C.c_int]
    ref.lib.sample_greedy.restype = C.c_int
    base = np.random.default_rng(1).standard_normal(4096).astype(np.float32)
    base[3000] = 40.0
    xs = []
    for idx, val in ((0, np.nan), (5, np.nan), (3000, np.nan), (0, np.inf)):
        x = base.copy()
        x[idx] = val
        xs.append(x)
    x = base.copy(); x[0] = np.nan; x[7] = np.inf; xs.append(x)
    xs.append(np.full(64, np.nan, np.float32))
    for x in xs:
        got = ref.lib.sample_greedy(x.ctypes.data_as(C.POINTER(C.c_float)), x.size)
        assert orc.argmax(x) == got
    assert orc.argmax(xs[0]) == 0 and orc.argmax(xs[1]) == 3000


def test_rope_closed_form(orc):
    """Adjacent-pair rotation by pos * theta^(-i/hd) (kernels_cpu.c:391-431)."""
    hd, theta = 128, 500000.0
    rng = np.random.default_rng(3)
    q = rng.standard_normal(2 * hd).astype(np.float32)
    k = rng.standard_normal(hd).astype(np.float32)
    i = np.arange(0, hd, 2)
    f = 1.0 / np.power(theta, i / hd)  # float64
    # at large positions one ulp of the fp32 frequency moves the angle by
    # ~pos * 2^-24 rad, so the bound widens with pos
    for pos, tol in ((7, 2e-6), (8191, 2e-3)):
        q2, k2 = orc.rope(q, k, 2, 1, hd, pos, theta)
        ang = pos * f
        c, s = np.cos(ang), np.sin(ang)
        for src, got in ((k, k2), (q[:hd], q2[:hd]), (q[hd:], q2[hd:])):
            x0, x1 = src[0::2].astype(np.float64), src[1::2].astype(np.float64)
            exp = np.empty(hd)
            exp[0::2], exp[1::2] = x0 * c - x1 * s, x0 * s + x1 * c
            assert np.abs(got - exp).max() < tol, pos


def test_attention_closed_form(orc):
    """softmax(q K^T / sqrt(hd)) V per head, GQA 4:1, fp64 brute force."""
    L, nkv, hd, nh, ms = 300, 2, 64, 8, 320
    kv = HostKV(1, nkv, hd, ms)
    kv.prefill(orc, S.TINY_TEST, L)
    q = orc.synth_normal(99, nh * hd)
    out = orc.attention(q, kv, 0, nh, L - 1)
    K = kv.view("k")[0].astype(np.float64)
    V = kv.view("v")[0].astype(np.float64)
    exp = np.zeros(nh * hd)
    for h in range(nh):
        g = h // (nh // nkv)
        s = K[g, :L] @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        exp[h * hd:(h + 1) * hd] = p @ V[g, :L]
    assert rel_l2(out, exp) < 1e-5


def test_kv_append_layout_and_wrap(orc):
    """Offset ((layer*n_kv + h)*max_seq + pos)*hd (kv_cache.c:90-93); pos wraps
    modulo max_seq (kv_cache.c:101)."""
    kv = HostKV(2, 2, 8, 16)
    from oracle import fptr
    import ctypes as C
    k = np.arange(16, dtype=np.float32) + 1
    v = -k
    for pos in (0, 5, 15, 16 + 3):
        assert orc.lib.orc_kv_append(C.byref(kv.s), 1, pos, fptr(k), fptr(v)) == 0
        p = pos % 16
        for h in range(2):
            assert np.array_equal(kv.view("k")[1, h, p], k[8 * h:8 * h + 8])
            assert np.array_equal(kv.view("v")[1, h, p], v[8 * h:8 * h + 8])
    assert not kv.view("k")[0].any()  # layer isolation (test_memory.c:151-190)
    assert orc.lib.orc_kv_append(C.byref(kv.s), 2, 0, fptr(k), fptr(v)) == -1


def test_lctx_image_layout(orc):
    """64-byte header, tokens, K all layers, V all layers (session.c:33-103)."""
    import ctypes as C
    from oracle import u8ptr
    kv = HostKV(2, 2, 8, 16)
    kv.prefill(orc, S.TINY_TEST, 10)
    toks = np.array([5, 6, 7], np.int32)
    n = orc.lib.orc_lctx_size(C.byref(kv.s), 3)
    assert n == 64 + 12 + 2 * kv.k.nbytes
    img = np.zeros(n, np.uint8)
    assert orc.lib.orc_lctx_write(C.byref(kv.s), 10, toks.ctypes.data_as(C.POINTER(C.c_int32)), 3,
                                  u8ptr(img), n) == 0
    hdr = img[:64].view(np.int32)
    # magic 0x5843544C stored little-endian: the first bytes read "LTCX"
    # (session.c:36 calls it "LCTX"; the bytes on disk are what counts)
    assert hdr[0] == 0x5843544C and bytes(img[:4]) == b"LTCX"
    assert list(hdr[1:8]) == [1, 2, 2, 8, 16, 10, 3]
    assert not img[32:64].any()
    assert np.array_equal(img[64:76].view(np.int32), toks)
    assert np.array_equal(img[76:76 + kv.k.nbytes].view(np.float32), kv.k)
    assert np.array_equal(img[76 + kv.k.nbytes:].view(np.float32), kv.v)


def test_lctx_bytes_match_reference(orc, ref, tmp_path):
    """The oracle's .lctx image is byte-identical to kv_cache_save's file."""
    import ctypes as C
    from oracle import u8ptr
    hm = HostModel(orc, S.TINY_TEST, 32)
    rm = RefModel(ref, hm)
    kv = hm.new_kv()
    kv.prefill(orc, S.TINY_TEST, 20)
    rm.load_kv(kv)
    toks = (C.c_int * 4)(3, 1, 4, 1)
    path = str(tmp_path / "s.lctx")
    assert ref.lib.kv_cache_save(rm.kv, C.byref(rm.mw.config), 32, 20, toks, 4, path.encode()) == 0
    n = orc.lib.orc_lctx_size(C.byref(kv.s), 4)
    img = np.zeros(n, np.uint8)
    t = np.array([3, 1, 4, 1], np.int32)
    orc.lib.orc_lctx_write(C.byref(kv.s), 20, t.ctypes.data_as(C.POINTER(C.c_int32)), 4, u8ptr(img), n)
    assert np.array_equal(np.fromfile(path, np.uint8), img)
    rm.close()


def test_prompt_cache_bytes_match_reference(orc, ref, tmp_path):
    """prompt_cache_save's file (session.c:192-237) is the oracle's .lctx
    image with current_pos = prefix_len and no tokens; prefix_len <= 0 is
    refused; prompt_cache_load returns prefix_len and the K/V."""
    import ctypes as C
    from oracle import u8ptr
    hm = HostModel(orc, S.TINY_TEST, 32)
    rm = RefModel(ref, hm)
    kv = hm.new_kv()
    kv.prefill(orc, S.TINY_TEST, 13)
    rm.load_kv(kv)
    path = str(tmp_path / "p.lctx")
    assert ref.lib.prompt_cache_save(rm.kv, C.byref(rm.mw.config), 32, 0, path.encode()) == -1
    assert ref.lib.prompt_cache_save(rm.kv, C.byref(rm.mw.config), 32, 13, path.encode()) == 0
    n = orc.lib.orc_lctx_size(C.byref(kv.s), 0)
    img = np.zeros(n, np.uint8)
    orc.lib.orc_lctx_write(C.byref(kv.s), 13, None, 0, u8ptr(img), n)
    assert np.array_equal(np.fromfile(path, np.uint8), img)
    for l in range(S.TINY_TEST.n_layers):
        rm.slab("k", l)[:] = 0
    got = C.c_int(-1)
    assert ref.lib.prompt_cache_load(rm.kv, C.byref(rm.mw.config), 32, C.byref(got), path.encode()) == 0
    assert got.value == 13
    n1 = kv.k.size // S.TINY_TEST.n_layers
    assert np.array_equal(rm.slab("k", 1), kv.k[n1:2 * n1])
    rm.close()


def test_forward_bitexact_vs_reference(orc, ref):
    """Whole decode steps: the oracle's logits equal the reference forward()'s."""
    hm = HostModel(orc, S.TINY_TEST, 64)
    kv = hm.new_kv()
    kv.prefill(orc, S.TINY_TEST, 24)
    rm = RefModel(ref, hm)
    rm.load_kv(kv)
    tok = 11
    for step in range(3):
        t1, l1, _ = hm.forward(kv, tok, 24 + step)
        t2, l2 = rm.forward(tok, 24 + step)
        assert t1 == t2 and np.array_equal(bits(l1), bits(l2))
        tok = t1
    for l in range(S.TINY_TEST.n_layers):
        assert np.array_equal(rm.slab("k", l), kv.k.reshape(S.TINY_TEST.n_layers, -1)[l])
    rm.close()


def test_synth_distributions(orc):
    z = orc.synth_normal(42, 200000).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01 and np.abs(z).max() <= 6
    w = orc.synth_quant(Q4_K, 9, 256, 256).reshape(256, 144)
    d = w[:, 0:2].copy().view(np.float16).astype(np.float64)
    assert d.min() >= 0.00099 and d.max() <= 0.0501
    w6 = orc.synth_quant(Q6_K, 9, 64, 256).reshape(64, 210)
    sc = w6[:, 192:208].view(np.int8)
    assert sc.min() >= -32 and sc.max() <= 31
