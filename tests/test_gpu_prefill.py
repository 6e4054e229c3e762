"""Prefill-chunk GEMM (config 5): Y = X W^T for T tokens on the bf16 matrix
cores.  Two references on the same seeded inputs:

* exact-input reference: X and the dequantized weights rounded to bf16 the
  way the kernel rounds them (dequant w = d sc q - dmin m rounded once to
  fp32, then to bf16 nearest-even), products and sums in fp64.  Only the
  kernel's fp32 accumulation order differs: tolerance 1e-5 relative L2.
  This is what pins indexing, operand layouts and the Q4_K decode.
* full-precision reference: fp64 GEMM of the fp32 X and the exactly
  dequantized weights (what the reference's T sequential fp32 matvecs
  approximate, engine.c:119-152).  bf16 inputs cost ~2^-9 relative per
  product: tolerance 1e-2 relative L2 (observed ~3e-3)."""
import numpy as np
import pytest

from guanaco_amd import spec as S
from util import dequant_q4k_f64, rel_l2

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
    import guanaco_amd.hip as H
    seed = (T << 20) ^ (N << 8) ^ K
    w = orc.synth_quant(S.Q4_K, seed, N, K)
    x = orc.synth_normal(seed + 1, T * K).reshape(T, K)
    r = orc.synth_normal(seed + 2, T * N).reshape(T, N)
    wd, xd = ctx.upload_weight(w), ctx.upload(x)
    yd = ctx.upload(r) if mode == 1 else ctx.alloc(4 * T * N)
    rc = H.lib.gq_hip_prefill_gemm_dev(ctx.h, S.Q4_K, mode, wd, N, K, xd.ptr, T, yd.ptr,
                                       yd.ptr if mode == 1 else None)
    assert rc == 0
    y = yd.download(count=T * N).reshape(T, N)
    base = r.astype(np.float64) if mode == 1 else 0.0
    exact_in = bf16_round(x).astype(np.float64) @ bf16_round(q4k_dequant_kernel_order(w, N, K)).astype(np.float64).T
    assert rel_l2(y, base + exact_in) < 1e-5
    full = x.astype(np.float64) @ dequant_q4k_f64(w, N, K).T
    e = rel_l2(y - base, full)
    assert e < 1e-2, e
    H.lib.gq_hip_free(ctx.h, wd)
    xd.free(), yd.free()


def test_prefill_gemm_rejects_bad_shapes(ctx):
    import guanaco_amd.hip as H
    buf = ctx.alloc(1 << 20)
    assert H.lib.gq_hip_prefill_gemm_dev(ctx.h, S.Q4_K, 0, buf.ptr, 100, 256, buf.ptr, 4, buf.ptr, None) != 0
    assert H.lib.gq_hip_prefill_gemm_dev(ctx.h, S.Q4_K, 0, buf.ptr, 128, 300, buf.ptr, 4, buf.ptr, None) != 0
    assert H.lib.gq_hip_prefill_gemm_dev(ctx.h, S.Q6_K, 0, buf.ptr, 128, 256, buf.ptr, 4, buf.ptr, None) != 0
    buf.free()
