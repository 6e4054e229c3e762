"""One decode step of a synthetic model in float64: how far an fp32 forward()
is from exact at that step.

The reference's forward() (engine.c:559-594, transformer_layer :353-554) and
the device path both round to fp32 in their own orders.  Where a step is ill
conditioned — two attention positions whose scores nearly tie while the
scores are large, or a top-2 logit gap near the rounding — the two orders
can differ by more than at a typical step.  This module computes the step in
float64 from the same inputs, so both fp32 results can be measured against
the exact one.

Inputs are the fp32 state the reference itself has at that step: the model's
weights (dequantized exactly: w = d*sc*q - dmin*m for Q4_K, d*sc*q for Q6_K,
d*q for Q8_0, all exact in float64), the KV rows of positions 0..pos-1 and
the RoPE (cos, sin) values of position pos as the reference computes them
in fp32 (kernels_cpu.c:408-413, the oracle's table from glibc powf/cosf/sinf).
Everything after that — RMSNorm, the projections, RoPE rotation, attention
with its softmax, SiLU, residual adds, final norm and LM head — is float64.

Test infrastructure (writes fixture values in make_golden.py); the product
never imports it.
"""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from util import DEQUANT  # noqa: E402  (closed-form dequantization, tests/util.py)


def _rmsnorm(x, w, eps):
    """cpu_rmsnorm (kernels_cpu.c:199-265) in float64: w * (x / sqrt(mean(x^2) + eps))."""
    return np.asarray(w, np.float64) * (x / np.sqrt(np.mean(x * x) + eps))


def _weight(dtype, data, rows, cols):
    return DEQUANT[dtype](data, rows, cols)


def forward_step(hm, kv, token, pos, lm_rows_chunk=8192):
    """Logits (float64, vocab) and per-layer hidden states (n_layers x hidden)
    of forward(token, pos) for the oracle HostModel `hm` over the fp32 cache
    `kv` holding positions 0..pos-1.  The cache is not modified."""
    s = hm.spec
    H, hd, nh, nkv = s.hidden, s.head_dim, s.n_heads, s.n_kv_heads
    g = nh // nkv
    eps = s.rms_eps
    # embedding row (engine.c:214-283): dequantized exactly
    bb = {2: 34, 4: 144, 5: 210}[s.embed_dtype]
    qk = 32 if s.embed_dtype == 2 else 256
    row_bytes = (H // qk) * bb
    x = _weight(s.embed_dtype, hm.embed[token * row_bytes:(token + 1) * row_bytes], 1, H)[0]
    cos32, sin32 = hm.orc.rope_table(hd, pos, s.rope_theta)
    c, sn = cos32.astype(np.float64), sin32.astype(np.float64)
    K = kv.view("k").astype(np.float64)[:, :, :pos + 1]
    V = kv.view("v").astype(np.float64)[:, :, :pos + 1]
    hidden = np.empty((s.n_layers, H))
    for l in range(s.n_layers):
        W = {k: _weight(dt, data, *s.shape(k)) for k, (dt, data) in hm.layer_w[l].items()}
        xn = _rmsnorm(x, hm.rms_att[l], eps)
        q, k, v = W["wq"] @ xn, W["wk"] @ xn, W["wv"] @ xn

        def rot(a):  # adjacent pairs (kernels_cpu.c:415-429)
            a = a.reshape(-1, hd // 2, 2)
            a0, a1 = a[..., 0].copy(), a[..., 1].copy()
            a[..., 0] = a0 * c - a1 * sn
            a[..., 1] = a0 * sn + a1 * c
            return a.reshape(-1, hd)

        q, k = rot(q), rot(k)
        Kl, Vl = K[l].copy(), V[l].copy()
        Kl[:, pos], Vl[:, pos] = k, v.reshape(nkv, hd)
        att = np.empty((nh, hd))
        for h in range(nh):
            sc = Kl[h // g] @ q[h] / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            att[h] = (p / p.sum()) @ Vl[h // g]
        x = x + W["wo"] @ att.reshape(-1)
        xn = _rmsnorm(x, hm.rms_ffn[l], eps)
        gt, up = W["wg"] @ xn, W["wu"] @ xn
        with np.errstate(over="ignore"):  # exp(-g) = inf for g << 0: silu(g) = -0.0, as it should
            x = x + W["wd"] @ (gt / (1.0 + np.exp(-gt)) * up)
        hidden[l] = x
        del W
    xn = _rmsnorm(x, hm.rms_final, eps)
    bb = {2: 34, 4: 144, 5: 210}[s.lm_head_dtype]
    qk = 32 if s.lm_head_dtype == 2 else 256
    row_bytes = (H // qk) * bb
    logits = np.empty(s.vocab)
    for r0 in range(0, s.vocab, lm_rows_chunk):
        r1 = min(s.vocab, r0 + lm_rows_chunk)
        logits[r0:r1] = _weight(s.lm_head_dtype, hm.lm_head[r0 * row_bytes:r1 * row_bytes], r1 - r0, H) @ xn
    return logits, hidden
