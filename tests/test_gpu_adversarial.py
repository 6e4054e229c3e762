"""The matvec kernels on adversarial activations, against the oracle's
restatement of the reference (quant_matvec_q4_k.c:65-140,
quant_matvec_q6_k.c:43-98; with the fused RMSNorm, kernels_cpu.c's
cpu_rmsnorm first, engine.c:356-366).

The matrix-core kernel ("mfma") turns each 256-value block of x (times the
norm weight) into exact int8 digit planes of a 22-bit fixed point scaled to
the block's largest magnitude, so these cases aim at that scaling:

* one element per block 1e4 times the rest (the small values keep 22 bits
  relative to the outlier);
* all-zero blocks (a zero block maximum);
* blocks whose maximum is subnormal, and an x that is subnormal throughout;
* a dynamic range of 1e-15 .. 1e15 across blocks (x^2 stays finite for the
  norm).

Bar: relative L2 and the largest row error (over the largest |y|) <= 1e-5,
as for every matvec test, on the vector-ALU path and the matrix-core path,
Q4_K and Q6_K, with and without the fused norm.

Non-finite policy: an inf or NaN anywhere in x makes every output row
non-finite (inf or NaN; which one, and the sign, are not specified), as it
does in the reference, where every row's dot product takes every column."""
import numpy as np
import pytest

from oracle import Q4_K, Q6_K
from util import rel_l2

pytestmark = pytest.mark.gpu

ROWS, COLS = 1024, 4096
TOL = 1e-5


def adversarial_x(orc, kind):
    x = orc.synth_normal(0xAD0 + len(kind), COLS).astype(np.float32)
    b = x.reshape(-1, 256)
    if kind == "outlier":
        b[::2, 37] *= np.float32(1e4)        # every other block: one element 1e4 x the rest
    elif kind == "zero_blocks":
        b[1::2] = 0.0                        # every other block all zero
        b[4] = 0.0
    elif kind == "subnormal_blocks":
        m = np.abs(b[1::3]).max(axis=1, keepdims=True)
        b[1::3] = (b[1::3] / m * np.float32(3e-39)).astype(np.float32)  # block max 3e-39 < 2^-126
        assert np.all(np.abs(b[1::3]).max(axis=1) < np.finfo(np.float32).tiny)
    elif kind == "all_subnormal":
        x = (x / np.abs(x).max() * np.float32(1e-38)).astype(np.float32)
        return x
    elif kind == "range":
        scale = np.float32(10.0) ** np.linspace(-15, 15, b.shape[0]).astype(np.float32)
        b *= scale[:, None]
    return x


KINDS = ["outlier", "zero_blocks", "subnormal_blocks", "all_subnormal", "range"]


@pytest.fixture(scope="module")
def weights(ctx, orc):
    out = {}
    for dt in (Q4_K, Q6_K):
        w = orc.synth_quant(dt, 0xAD5 + dt, ROWS, COLS)
        out[dt] = (w, ctx.upload_weight(w))
    nw = orc.synth_norm_weight(0xAD7, COLS)
    return out, nw, ctx.upload(nw)


def _run(ctx, dt, wd, x, norm, nwb, path):
    import guanaco_amd.hip as H
    xb, yb = ctx.upload(x), ctx.alloc(4 * ROWS)
    with H.matvec_path(path):
        if norm:
            ctx.matvec_norm_dev(dt, wd, ROWS, COLS, xb, nwb, 1e-6, yb)
        else:
            ctx.matvec_dev(dt, wd, ROWS, COLS, xb, yb)
        ctx.sync()
    y = yb.download(count=ROWS)
    xb.free(), yb.free()
    return y


@pytest.mark.parametrize("path", ["valu", "mfma"])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
@pytest.mark.parametrize("kind", KINDS)
def test_matvec_adversarial_x(ctx, orc, weights, kind, dt, norm, path):
    ws, nw, nwb = weights
    w, wd = ws[dt]
    x = adversarial_x(orc, kind)
    y = _run(ctx, dt, wd, x, norm, nwb, path)
    xr = orc.rmsnorm(x, nw, 1e-6) if norm else x
    ref = orc.matvec(dt, w, ROWS, COLS, xr)
    assert np.all(np.isfinite(ref)) and np.all(np.isfinite(y)), kind
    assert rel_l2(y, ref) < TOL, (kind, rel_l2(y, ref))
    assert np.abs(y - ref).max() <= TOL * np.abs(ref).max(), kind


@pytest.mark.parametrize("path", ["valu", "mfma"])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
def test_matvec_nonfinite_x_policy(ctx, orc, weights, bad, dt, norm, path):
    ws, nw, nwb = weights
    w, wd = ws[dt]
    x = orc.synth_normal(0xAD9, COLS).astype(np.float32)
    x[1000] = bad
    y = _run(ctx, dt, wd, x, norm, nwb, path)
    xr = orc.rmsnorm(x, nw, 1e-6) if norm else x
    ref = orc.matvec(dt, w, ROWS, COLS, xr)
    assert not np.isfinite(ref).any()  # the reference: every row non-finite
    assert not np.isfinite(y).any(), f"{np.isfinite(y).sum()} finite rows"
