"""GPU parity of the matvec and glue kernels through the C ABI, against the
CPU oracle (pinned to the reference in test_oracle.py) on the same seeded
inputs.  Tolerance: relative L2 <= 1e-5 for matvecs (the north star allows
1e-3 per layer; a correct kernel differs from the CPU order by ~1e-7)."""
import ctypes as C

import numpy as np
import pytest

from oracle import F32, Q4_K, Q6_K, Q8_0, OrcTensor, fptr, u8ptr
from util import bits, rel_l2

pytestmark = pytest.mark.gpu

MV_TOL = 1e-5


@pytest.mark.parametrize("dt", [Q4_K, Q6_K, Q8_0])
def test_device_synth_matches_host(ctx, orc, dt):
    rows, cols = (37, 5632) if dt != Q8_0 else (37, 1024)
    seed = 0xABCDEF + dt
    dev = ctx.synth_quant(dt, rows, cols, seed)
    host = orc.synth_quant(dt, seed, rows, cols)
    assert np.array_equal(dev.download(np.uint8, host.size), host)
    dev.free()


def test_device_synth_normal_matches_host(ctx, orc):
    n = 100003
    a = ctx.synth_normal(n, 99)
    b = ctx.synth_norm_weight(n, 98)
    assert np.array_equal(bits(a.download(count=n)), bits(orc.synth_normal(99, n)))
    assert np.array_equal(bits(b.download(count=n)), bits(orc.synth_norm_weight(98, n)))


SHAPES = [
    (Q4_K, 1, 256), (Q4_K, 8, 512), (Q4_K, 64, 1024), (Q4_K, 37, 5632), (Q4_K, 1024, 4096),
    (Q4_K, 4096, 4096), (Q4_K, 301, 14336), (Q4_K, 5632, 2048),
    (Q6_K, 1, 256), (Q6_K, 8, 512), (Q6_K, 64, 1024), (Q6_K, 37, 5632), (Q6_K, 1024, 4096),
    (Q6_K, 4096, 4096), (Q6_K, 301, 14336), (Q6_K, 2048, 5632),
    (Q8_0, 1, 32), (Q8_0, 8, 512), (Q8_0, 33, 1024), (Q8_0, 64, 4096),
    # rows longer than 16384 columns: 1024-thread groups (28672: an ff-28672
    # down projection), then several column tiles per lane (40960, 65536)
    (Q4_K, 64, 28672), (Q6_K, 64, 28672), (Q8_0, 40, 28672),
    (Q4_K, 33, 65536), (Q6_K, 48, 40960), (Q8_0, 24, 40960),
]


@pytest.mark.parametrize("path", ["auto", "valu", "mfma"])
@pytest.mark.parametrize("dt,rows,cols", SHAPES)
def test_matvec_vs_oracle(ctx, orc, dt, rows, cols, path):
    import guanaco_amd.hip as H
    seed = (dt << 20) ^ (rows << 8) ^ cols
    w = orc.synth_quant(dt, seed, rows, cols)
    x = orc.synth_normal(seed + 1, cols)
    wd = ctx.upload_weight(w)
    with H.matvec_path(path):
        rc, y = ctx.matvec_host(dt, wd, rows, cols, x, byte_size=w.nbytes)
    assert rc == 0
    ref = orc.matvec(dt, w, rows, cols, x)
    assert rel_l2(y, ref) < MV_TOL
    # every row, not just the norm: no row may be dropped or swapped
    scale = np.abs(ref).max() + 1e-30
    assert np.abs(y - ref).max() / scale < 1e-5
    C.CDLL(None)  # keep ctypes imported for linters
    __import__("guanaco_amd.hip").hip.lib.gq_hip_free(ctx.h, wd)


@pytest.mark.parametrize("dt,rows,cols", [(Q6_K, 32776, 4096), (Q4_K, 32768, 8192)])
def test_matvec_mfma_many_stages(ctx, orc, dt, rows, cols):
    """Matrix-core launches whose workgroups run 16 or more stages (the
    LM head's shape class) drop the per-stage barrier: each wave copies only
    the blocks it computes, and the tiles are finished after the loop.  Q6_K
    32776 x 4096 (two chunks a row, 8 tiles a workgroup, the last tile
    half full) and Q4_K 32768 x 8192 (two chunks, 8 tiles) against the
    oracle, every row."""
    import guanaco_amd.hip as H
    seed = 0x5A6E ^ (dt << 20) ^ rows
    w = orc.synth_quant(dt, seed, rows, cols)
    x = orc.synth_normal(seed + 1, cols)
    wd = ctx.upload_weight(w)
    with H.matvec_path("mfma"):
        rc, y = ctx.matvec_host(dt, wd, rows, cols, x, byte_size=w.nbytes)
    assert rc == 0
    ref = orc.matvec(dt, w, rows, cols, x)
    assert rel_l2(y, ref) < MV_TOL
    assert np.abs(y - ref).max() / (np.abs(ref).max() + 1e-30) < 1e-5
    H.lib.gq_hip_free(ctx.h, wd)


# Rows of 32 .. 4096 columns: a 256-thread workgroup holds 32 .. 2 row groups
# (8- to 128-lane groups; below 64 lanes a group is part of a wave), which
# share x times the norm weights through LDS; Q8_0 rows of 9 and 1 units
# leave lanes of every group idle.
NORM_SHAPES = [
    (Q4_K, 64, 256), (Q4_K, 48, 512), (Q4_K, 96, 1024), (Q4_K, 40, 2048), (Q4_K, 36, 4096),
    (Q6_K, 64, 512), (Q6_K, 40, 2048), (Q8_0, 40, 32), (Q8_0, 37, 288), (Q8_0, 24, 1024),
]


@pytest.mark.parametrize("dt,rows,cols", NORM_SHAPES)
def test_matvec_norm_vs_oracle(ctx, orc, dt, rows, cols):
    """The fused RMSNorm prologue (kernels_cpu.c:242-253, then the matvec of
    the normalised x) at every row-group count, on the vector-ALU path."""
    import guanaco_amd.hip as H
    seed = 0x5E0 + 7 * dt + cols
    w = orc.synth_quant(dt, seed, rows, cols)
    x = orc.synth_normal(seed + 1, cols)
    nw = orc.synth_norm_weight(seed + 2, cols)
    wd = ctx.upload_weight(w)
    xb, nwb, yb = ctx.upload(x), ctx.upload(nw), ctx.alloc(4 * rows)
    with H.matvec_path("valu"):
        ctx.matvec_norm_dev(dt, wd, rows, cols, xb, nwb, 1e-5, yb)
        ctx.sync()
    y = yb.download(count=rows)
    ref = orc.matvec(dt, w, rows, cols, orc.rmsnorm(x, nw, 1e-5))
    assert rel_l2(y, ref) < MV_TOL
    assert np.abs(y - ref).max() <= MV_TOL * np.abs(ref).max()
    xb.free(), nwb.free(), yb.free()
    H.lib.gq_hip_free(ctx.h, wd)


def test_matvec_error_codes(ctx):
    """The vtable convention (quant_matvec_q4_k.c:143-158, test_backend.c:71-86):
    NULL/zeroed tensor -1, cols % 256 -2, short byte_size -3."""
    w = np.zeros(144 * 4, np.uint8)
    wd = ctx.upload_weight(w)
    x = np.zeros(1024, np.float32)
    assert ctx.matvec_host(Q4_K, None, 1, 1024, x)[0] == -1
    assert ctx.matvec_host(99, wd, 1, 1024, x)[0] == -1
    assert ctx.matvec_host(Q4_K, wd, 1, 1000, x)[0] == -2
    assert ctx.matvec_host(Q4_K, wd, 1, 1024, x, byte_size=144 * 4 - 1)[0] == -3
    assert ctx.matvec_host(Q4_K, wd, 1, 1024, x, byte_size=144 * 4)[0] == 0
    assert ctx.matvec_host(Q4_K, wd, 0, 1024, x)[0] == -1


def test_q4k_known_answers(ctx):
    """test_quant.c:94-139 (384) through the GPU kernel."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[4:16] = 1
    blk[16:] = 0x12
    wd = ctx.upload_weight(blk)
    rc, y = ctx.matvec_host(Q4_K, wd, 1, 256, np.ones(256, np.float32))
    assert rc == 0 and abs(y[0] - 384.0) < 1e-4


def test_rmsnorm(ctx, orc):
    n = 4096
    x = orc.synth_normal(3, n) * np.float32(7.0)
    w = orc.synth_norm_weight(4, n)
    xb, wb, ob = ctx.upload(x), ctx.upload(w), ctx.alloc(4 * n)
    ctx.rmsnorm_dev(xb, wb, ob, n, 1e-6)
    assert rel_l2(ob.download(), orc.rmsnorm(x, w, 1e-6)) < 1e-6


@pytest.mark.parametrize("dt", [Q4_K, Q8_0, F32])
def test_embedding_row_bitexact(ctx, orc, dt):
    """Embedding dequant rounds like engine.c:241-276: bit-identical rows."""
    vocab, H = 50, 512
    if dt == F32:
        table = orc.synth_normal(5, vocab * H)
        raw = table.view(np.uint8)
    else:
        raw = orc.synth_quant(dt, 5, vocab, H)
    td = ctx.upload_weight(raw)
    t = OrcTensor(dt, vocab, H, u8ptr(raw), raw.nbytes)
    ob = ctx.alloc(4 * H)
    for tok in (0, 17, vocab - 1):
        ctx.embed_dev(dt, td, H, tok, ob)
        exp = np.empty(H, np.float32)
        orc.lib.orc_embed(C.byref(t), tok, fptr(exp))
        assert np.array_equal(bits(ob.download()), bits(exp)), tok


def test_argmax_first_max(ctx):
    """Ties go to the lowest index (tokenizer.c:175-185)."""
    assert ctx.argmax_dev(ctx.upload(np.array([3, 1, 3, 2], np.float32)), 4) == 0
    x = np.random.default_rng(0).standard_normal(128256).astype(np.float32)
    x[[70000, 5000, 120000]] = 50.0
    assert ctx.argmax_dev(ctx.upload(x), x.size) == 5000
    x[:] = -np.inf
    assert ctx.argmax_dev(ctx.upload(x), x.size) == 0


def test_argmax_nan(ctx, orc):
    """NaN logits as sample_greedy (tokenizer.c:175-185) treats them: a NaN at
    index 0 is never replaced (no value compares greater), a NaN anywhere
    else is never taken.  Checked against the oracle's restatement of that
    scan, which test_oracle pins against the compiled reference."""
    base = np.random.default_rng(1).standard_normal(128256).astype(np.float32)
    base[70000] = 40.0
    cases = []
    x = base.copy(); x[0] = np.nan; cases.append((x, 0))
    x = base.copy(); x[0] = np.nan; x[9] = np.inf; cases.append((x, 0))
    x = base.copy(); x[5000] = np.nan; cases.append((x, 70000))
    x = base.copy(); x[70000] = np.nan; x[[3, 99999]] = 39.0; cases.append((x, 3))
    x = base.copy(); x[1:] = np.nan; cases.append((x, 0))
    x = np.full(128256, np.nan, np.float32); x[64000] = -1.0; cases.append((x, 0))
    for x, want in cases:
        assert orc.argmax(x) == want
        assert ctx.argmax_dev(ctx.upload(x), x.size) == want


def test_silu_mul(ctx, orc):
    n = 14336
    g = orc.synth_normal(1, n) * np.float32(4)
    u = orc.synth_normal(2, n)
    gb, ub = ctx.upload(g), ctx.upload(u)
    ctx.silu_mul_dev(gb, ub, n)
    gg = g.copy()
    orc.lib.orc_silu(fptr(gg), n)
    assert rel_l2(gb.download(), gg * u) < 1e-6


def test_copy_kernel(ctx):
    """gq_hip_copy_dev: the plain copy used to scale the HBM byte counters."""
    import guanaco_amd.hip as H
    n = (3 << 20) + 48
    src = ctx.upload(np.arange(n // 4, dtype=np.float32))
    dst = ctx.alloc(n)
    assert H.lib.gq_hip_copy_dev(ctx.h, dst.ptr, src.ptr, n) == 0
    assert np.array_equal(dst.download(count=n // 4), np.arange(n // 4, dtype=np.float32))
    assert H.lib.gq_hip_copy_dev(ctx.h, dst.ptr, src.ptr, 8) == -1  # not a multiple of 16
    src.free(), dst.free()


def test_time_read_floor_kernel(ctx):
    """gq_hip_time_read: the read-only streaming kernel behind the single-
    launch floor of the profiles.  It times launches over rotating regions
    (a 3 MiB + 48 B region, not a multiple of the grid's pass) and rejects
    sizes that are not multiples of 16 and regions that overlap."""
    import guanaco_amd.hip as H
    buf = ctx.upload(np.arange(4 << 20, dtype=np.float32))  # 16 MiB
    n = (3 << 20) + 48
    ms = H.lib.gq_hip_time_read(ctx.h, buf.ptr, n, 4 << 20, 4, 8)
    assert ms > 0, ms
    assert H.lib.gq_hip_time_read(ctx.h, buf.ptr, 1000, 0, 1, 4) < 0           # not a multiple of 16
    assert H.lib.gq_hip_time_read(ctx.h, buf.ptr, 4 << 20, 2 << 20, 2, 4) < 0  # regions overlap
    assert np.array_equal(buf.download(count=16), np.arange(16, dtype=np.float32))  # nothing stored
    buf.free()
    # one pass at any size: 272 MiB takes 8704 workgroups, more than the
    # 4096-entry sink the (never taken) marker store indexes modulo
    big = ctx.alloc(272 << 20)
    assert H.lib.gq_hip_time_read(ctx.h, big.ptr, 272 << 20, 0, 1, 2) > 0
    big.free()
