import numpy as np


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def f16(x):
    return np.float16(x).view(np.uint16)


def q4k_block(d, dmin, scales, qs):
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(dmin).tobytes(), np.uint8)
    b[4:16] = scales
    b[16:144] = qs
    return b


def dequant_q4k_f64(w, rows, cols):
    """Closed form of the Q4_K format (no reference code): w = d*sc*q - dmin*m."""
    nb = cols // 256
    blk = w.reshape(rows, nb, 144)
    d = blk[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dm = blk[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    s = blk[:, :, 4:16].astype(np.int64)
    sc = np.zeros((rows, nb, 8)); mn = np.zeros((rows, nb, 8))
    for j in range(8):
        if j < 4:
            sc[..., j] = s[..., j] & 63
            mn[..., j] = s[..., j + 4] & 63
        else:
            sc[..., j] = (s[..., j + 4] & 15) | ((s[..., j - 4] >> 6) << 4)
            mn[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    qs = blk[:, :, 16:].astype(np.int64).reshape(rows, nb, 4, 32)
    out = np.zeros((rows, nb, 4, 64))
    for c in range(4):
        out[:, :, c, :32] = d[..., None] * sc[:, :, 2 * c, None] * (qs[:, :, c] & 15) - dm[..., None] * mn[:, :, 2 * c, None]
        out[:, :, c, 32:] = d[..., None] * sc[:, :, 2 * c + 1, None] * (qs[:, :, c] >> 4) - dm[..., None] * mn[:, :, 2 * c + 1, None]
    return out.reshape(rows, cols)


def dequant_q6k_f64(w, rows, cols):
    """Closed form of the Q6_K format: w = d*sc*(q6-32)."""
    nb = cols // 256
    blk = w.reshape(rows, nb, 210)
    ql = blk[..., 0:128].astype(np.int64)
    qh = blk[..., 128:192].astype(np.int64)
    sc = blk[..., 192:208].view(np.int8).astype(np.float64)
    d = blk[..., 208:210].copy().view(np.float16)[..., 0].astype(np.float64)
    out = np.zeros((rows, nb, 256))
    for h in range(2):
        for l in range(32):
            s = l // 16
            a, b, hh = ql[..., 64 * h + l], ql[..., 64 * h + l + 32], qh[..., 32 * h + l]
            q = [(a & 15) | ((hh & 3) << 4), (b & 15) | (((hh >> 2) & 3) << 4),
                 (a >> 4) | (((hh >> 4) & 3) << 4), (b >> 4) | (((hh >> 6) & 3) << 4)]
            for k in range(4):
                out[..., 128 * h + l + 32 * k] = d * sc[..., 8 * h + s + 2 * k] * (q[k] - 32)
    return out.reshape(rows, cols)


def dequant_q8_0_f64(w, rows, cols):
    nb = cols // 32
    blk = w.reshape(rows, nb, 34)
    d = blk[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    q = blk[..., 2:].view(np.int8).astype(np.float64)
    return (d[..., None] * q).reshape(rows, cols)


DEQUANT = {4: dequant_q4k_f64, 5: dequant_q6k_f64, 2: dequant_q8_0_f64}
