"""Vectorised numpy decoders of the eight block layouts, independent of the oracle's C code.

Each decoder returns, per weight element, integer codes such that the weight equals
    d * sc * q - dmin * m      (Q4_K, Q5_K, Q2_K)   or   d * sc * q      (Q6_K: q already minus 32; Q3_K: q in -4..3,
    sc already minus 32; Q4_0/Q5_0/Q8_0: sc = 1)
and the tests pin the decoders by rebuilding the reference's dequantized floats (es_dequant_row) bit for bit.
The integer block dot of a weight block against int8 activations is then sum(sc*q*y) (and sum(m*y) for the mins),
computed here in int64 by brute force.
"""
import numpy as np


def _f16(u16):
    return np.asarray(u16, np.uint16).view(np.float16).astype(np.float32)


def decode(t, W, cols):
    """-> dict(q [rows, cols] int64, sc [rows, cols] int64, m [rows, cols] int64, d [rows, nb] f32, dmin [rows, nb])"""
    W = np.asarray(W, np.uint8)
    if t == 8:   # Q8_0: d f16, int8 qs[32]
        B = W.reshape(-1, 34)
        d = _f16(B[:, 0:2].copy().view(np.uint16)[:, 0])
        q = B[:, 2:34].copy().view(np.int8).astype(np.int64)
        rows = W.size // (cols // 32 * 34)
        return dict(q=q.reshape(rows, cols), sc=np.ones((rows, cols), np.int64), m=np.zeros((rows, cols), np.int64),
                    d=d.reshape(rows, -1), dmin=np.zeros((rows, cols // 32), np.float32), bs=32)
    if t in (2, 6):
        bb = 18 if t == 2 else 22
        B = W.reshape(-1, bb)
        d = _f16(B[:, 0:2].copy().view(np.uint16)[:, 0])
        qs = B[:, 2:18] if t == 2 else B[:, 6:22]
        nib = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int64)   # elements 0..15 low, 16..31 high
        if t == 6:
            qh = B[:, 2:6].copy().view(np.uint32)[:, 0].astype(np.int64)
            bits = (qh[:, None] >> np.arange(32)[None, :]) & 1
            q = (nib | (bits << 4)) - 16
        else:
            q = nib - 8
        rows = W.size // (cols // 32 * bb)
        return dict(q=q.reshape(rows, cols), sc=np.ones((rows, cols), np.int64), m=np.zeros((rows, cols), np.int64),
                    d=d.reshape(rows, -1), dmin=np.zeros((rows, cols // 32), np.float32), bs=32)
    if t in (12, 13):   # Q4_K, Q5_K (Q4_K plus a fifth bit per element from qh)
        B = W.reshape(-1, 144 if t == 12 else 176)
        d = _f16(B[:, 0:2].copy().view(np.uint16)[:, 0])
        dm = _f16(B[:, 2:4].copy().view(np.uint16)[:, 0])
        s = B[:, 4:16].astype(np.int64)
        sc = np.zeros((B.shape[0], 8), np.int64)
        mn = np.zeros((B.shape[0], 8), np.int64)
        sc[:, :4] = s[:, 0:4] & 63
        mn[:, :4] = s[:, 4:8] & 63
        sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
        mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
        qs = B[:, 16:144] if t == 12 else B[:, 48:176]
        qs = qs.reshape(-1, 4, 32).astype(np.int64)
        lo, hi = qs & 15, qs >> 4
        if t == 13:   # qh bit 2c of byte l: element 64c + l; bit 2c + 1: element 64c + 32 + l
            qh = B[:, 16:48].astype(np.int64)[:, None, :]
            c = np.arange(4)[None, :, None]
            lo = lo | (((qh >> (2 * c)) & 1) << 4)
            hi = hi | (((qh >> (2 * c + 1)) & 1) << 4)
        q = np.stack([lo, hi], axis=2).reshape(-1, 256)   # chunk c: 32 low then 32 high
        scx = np.repeat(sc, 32, axis=1)
        mx = np.repeat(mn, 32, axis=1)
    elif t == 14:   # Q6_K
        B = W.reshape(-1, 210)
        d = _f16(B[:, 208:210].copy().view(np.uint16)[:, 0])
        dm = np.zeros_like(d)
        ql = B[:, :128].reshape(-1, 2, 2, 32).astype(np.int64)      # half, (first/second 32 bytes), l
        qh = B[:, 128:192].reshape(-1, 2, 32).astype(np.int64)
        v = np.zeros((B.shape[0], 2, 4, 32), np.int64)
        for k in range(4):
            low = (ql[:, :, k & 1, :] >> (4 * (k >> 1))) & 15
            v[:, :, k, :] = (low | (((qh >> (2 * k)) & 3) << 4)) - 32
        q = v.reshape(-1, 256)
        scx = np.repeat(B[:, 192:208].view(np.int8).astype(np.int64), 16, axis=1)
        mx = np.zeros_like(scx)
    elif t == 11:   # Q3_K: group g = 8n + 2j + half, 16 elements; bits 2j of qs[32n + 16 half + l], hmask bit 4n + j
        B = W.reshape(-1, 110)
        d = _f16(B[:, 108:110].copy().view(np.uint16)[:, 0])
        dm = np.zeros_like(d)
        hm = B[:, 0:32].reshape(-1, 2, 16).astype(np.int64)
        qs = B[:, 32:96].reshape(-1, 2, 2, 16).astype(np.int64)     # n, half, l
        v = np.zeros((B.shape[0], 2, 4, 2, 16), np.int64)           # n, j, half, l
        for n in range(2):
            for j in range(4):
                v[:, n, j] = ((qs[:, n] >> (2 * j)) & 3) - np.where((hm >> (4 * n + j)) & 1, 0, 4)
        q = v.reshape(-1, 256)
        s = B[:, 96:108].astype(np.int64)
        lo = np.concatenate([s[:, 0:8] & 15, s[:, 0:8] >> 4], axis=1)
        g = np.arange(16)
        hi = (s[:, 8 + (g & 3)] >> (2 * (g >> 2))) & 3
        scx = np.repeat((lo | (hi << 4)) - 32, 16, axis=1)
        mx = np.zeros_like(scx)
    elif t == 10:   # Q2_K
        B = W.reshape(-1, 84)
        d = _f16(B[:, 80:82].copy().view(np.uint16)[:, 0])
        dm = _f16(B[:, 82:84].copy().view(np.uint16)[:, 0])
        qs = B[:, 16:80].reshape(-1, 2, 2, 16).astype(np.int64)     # half, part, l
        v = np.zeros((B.shape[0], 2, 4, 2, 16), np.int64)           # half, shift, part, l
        for s in range(4):
            v[:, :, s, :, :] = (qs >> (2 * s)) & 3
        q = v.reshape(-1, 256)
        sc8 = B[:, :16].astype(np.int64)
        scx = np.repeat(sc8 & 15, 16, axis=1)
        mx = np.repeat(sc8 >> 4, 16, axis=1)
    else:
        raise ValueError(t)
    nb = cols // 256
    rows = q.shape[0] // nb
    return dict(q=q.reshape(rows, cols), sc=scx.reshape(rows, cols), m=mx.reshape(rows, cols),
                d=d.reshape(rows, nb), dmin=dm.reshape(rows, nb), bs=256)


def dequant_like_reference(t, dec):
    """float weights with the reference's per-format float formula (src/es_quant.c:117-181, 425-472, es_q2k.c:88-100)"""
    bs = dec["bs"]
    d = np.repeat(dec["d"], bs, axis=1)
    dm = np.repeat(dec["dmin"], bs, axis=1)
    q, sc, m = dec["q"], dec["sc"], dec["m"]
    if t in (2, 6, 8):
        return q.astype(np.float32) * d
    if t in (11, 14):
        return (d * sc.astype(np.float32)) * q.astype(np.float32)
    return (d * sc.astype(np.float32)) * q.astype(np.float32) - dm * m.astype(np.float32)


def int_dots(dec, y8):
    """brute-force per-block integer dots of every row against one activation's int8 values y8 [cols]"""
    bs = dec["bs"]
    y = np.asarray(y8, np.int64)[None, :]
    rows, cols = dec["q"].shape
    dot = (dec["sc"] * dec["q"] * y).reshape(rows, cols // bs, bs).sum(axis=2)
    mins = (dec["m"] * y).reshape(rows, cols // bs, bs).sum(axis=2)
    return dot, mins
