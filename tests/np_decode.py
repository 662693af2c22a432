"""Independent numpy decoder of the thirteen GGUF block layouts, written from the
byte-layout descriptions (element order, nibble order, scale packing) rather than from any
kernel.

decode(w, qtype, n, k) -> (q, scale, wmin), each (n, k):
    weight value = scale * q - wmin      (float64 exact; q is the stored integer)
Q4_0 / Q5_0 / Q6_K / Q3_K return q with their offsets (-8, -16, -32, -4) already applied;
F32 / F16 return the values themselves as q (scale 1, wmin 0).
"""
from __future__ import annotations

import numpy as np

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = (
    0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14)
TS = {F32: 4, F16: 2, Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34, Q8_1: 36, Q2_K: 84,
      Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}
BS = {F32: 1, F16: 1, Q4_0: 32, Q4_1: 32, Q5_0: 32, Q5_1: 32, Q8_0: 32, Q8_1: 32, Q2_K: 256,
      Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}


def _f16(b: np.ndarray) -> np.ndarray:
    """(nblk, 2) little-endian fp16 bytes -> (nblk,) float64."""
    return np.ascontiguousarray(b).view(np.float16)[:, 0].astype(np.float64)


def _k4_scales(sc12: np.ndarray):
    """(nblk, 12) packed bytes -> (nblk, 8) scales and mins, 6 bits each.
    Sub-blocks 0-3: low 6 bits of bytes 0-3 (scale) and 4-7 (min). Sub-blocks 4-7: low /
    high nibble of bytes 8-11 give the low 4 bits of scale / min, and the top two bits of
    bytes 0-3 (scale) and 4-7 (min) give bits 4-5."""
    s = sc12.astype(np.int64)
    sc = np.zeros((s.shape[0], 8), np.int64)
    mn = np.zeros((s.shape[0], 8), np.int64)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, mn


def decode(w: np.ndarray, qtype: int, n: int, k: int):
    nb = k // BS[qtype]
    blk = np.asarray(w, np.uint8)[: n * nb * TS[qtype]].reshape(n * nb, TS[qtype])
    nblk = blk.shape[0]
    if qtype == Q8_0:
        d = _f16(blk[:, 0:2])
        q = blk[:, 2:34].view(np.int8).astype(np.int64)
        scale = np.repeat(d[:, None], 32, axis=1)
        wmin = np.zeros_like(scale)
    elif qtype in (Q4_0, Q5_0):
        d = _f16(blk[:, 0:2])
        qs = blk[:, 6:22] if qtype == Q5_0 else blk[:, 2:18]
        q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int64)  # elems 0-15, 16-31
        if qtype == Q5_0:
            qh = blk[:, 2:6].astype(np.uint32)
            bits = qh[:, 0] | (qh[:, 1] << 8) | (qh[:, 2] << 16) | (qh[:, 3] << 24)
            hb = (bits[:, None] >> np.arange(32, dtype=np.uint32)[None, :]) & 1
            q = (q | (hb.astype(np.int64) << 4)) - 16
        else:
            q = q - 8
        scale = np.repeat(d[:, None], 32, axis=1)
        wmin = np.zeros_like(scale)
    elif qtype in (Q4_K, Q5_K):
        d = _f16(blk[:, 0:2])
        dmin = _f16(blk[:, 2:4])
        sc, mn = _k4_scales(blk[:, 4:16])
        qs = blk[:, 48:176] if qtype == Q5_K else blk[:, 16:144]
        q = np.zeros((nblk, 256), np.int64)
        for c in range(4):  # 32-byte chunk c: low nibbles -> sub-block 2c, high -> 2c + 1
            q[:, 64 * c: 64 * c + 32] = qs[:, 32 * c: 32 * c + 32] & 15
            q[:, 64 * c + 32: 64 * c + 64] = qs[:, 32 * c: 32 * c + 32] >> 4
        if qtype == Q5_K:
            qh = blk[:, 16:48].astype(np.int64)  # bit j of qh[l] -> bit 4 of elem 32j + l
            for j in range(8):
                q[:, 32 * j: 32 * j + 32] |= ((qh >> j) & 1) << 4
        scale = (d[:, None] * np.repeat(sc, 32, axis=1))
        wmin = (dmin[:, None] * np.repeat(mn, 32, axis=1))
    elif qtype == Q6_K:
        ql = blk[:, 0:128].astype(np.int64)
        qh = blk[:, 128:192].astype(np.int64)
        sc = blk[:, 192:208].view(np.int8).astype(np.int64)
        d = _f16(blk[:, 208:210])
        q = np.zeros((nblk, 256), np.int64)
        for g in range(2):      # 128-element halves
            for i in range(4):  # 32-element sub-blocks
                low = ql[:, 64 * g + 32 * (i & 1): 64 * g + 32 * (i & 1) + 32]
                low = (low & 15) if i < 2 else (low >> 4)
                hi = (qh[:, 32 * g: 32 * g + 32] >> (2 * i)) & 3
                q[:, 128 * g + 32 * i: 128 * g + 32 * i + 32] = (low | (hi << 4)) - 32
        scale = d[:, None] * np.repeat(sc, 16, axis=1)
        wmin = np.zeros_like(scale)
    elif qtype in (F32, F16):
        q = blk.view(np.float32 if qtype == F32 else np.float16)[:, 0].astype(np.float64)
        q = q[:, None]
        scale = np.ones_like(q)
        wmin = np.zeros_like(q)
    elif qtype == Q8_1:  # [d][s][qs i8 x32]; s only serves dot products
        d = _f16(blk[:, 0:2])
        q = blk[:, 4:36].view(np.int8).astype(np.int64)
        scale = np.repeat(d[:, None], 32, axis=1)
        wmin = np.zeros_like(scale)
    elif qtype in (Q4_1, Q5_1):  # value = d * q + m
        d, m = _f16(blk[:, 0:2]), _f16(blk[:, 2:4])
        qs = blk[:, 8:24] if qtype == Q5_1 else blk[:, 4:20]
        q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int64)
        if qtype == Q5_1:
            qh = blk[:, 4:8].copy().view("<u4")[:, 0].astype(np.int64)
            q |= ((qh[:, None] >> np.arange(32)[None, :]) & 1) << 4
        scale = np.repeat(d[:, None], 32, axis=1)
        wmin = -np.repeat(m[:, None], 32, axis=1)
    elif qtype == Q2_K:  # [scales 16][qs 64][d][dmin]
        d, dmin = _f16(blk[:, 80:82]), _f16(blk[:, 82:84])
        scb = blk[:, 0:16].astype(np.int64)
        qs = blk[:, 16:80].astype(np.int64)
        e = np.arange(256)
        h, j, l = e // 128, (e % 128) // 32, e % 32
        q = (qs[:, 32 * h + l] >> (2 * j)) & 3              # (nblk, 256) by fancy indexing
        sidx = 8 * h + 2 * j + (l >= 16)
        scale = d[:, None] * (scb[:, sidx] & 15)
        wmin = dmin[:, None] * (scb[:, sidx] >> 4)
    elif qtype == Q3_K:  # [hmask 32][qs 64][scales 12][d]
        d = _f16(blk[:, 108:110])
        hm = blk[:, 0:32].astype(np.int64)
        qs = blk[:, 32:96].astype(np.int64)
        # the 16 six-bit scales: bytes 0-7 carry the low nibbles (scales 0-7) and high
        # nibbles (scales 8-15); byte 8 + (i mod 4) carries bits 4-5 of scales i, i+4, i+8,
        # i+12 in its bit pairs 0-1, 2-3, 4-5, 6-7
        raw = blk[:, 96:108].astype(np.int64)
        low = np.concatenate([raw[:, 0:8] & 15, raw[:, 0:8] >> 4], axis=1)
        top = np.concatenate([(raw[:, 8:12] >> (2 * g)) & 3 for g in range(4)], axis=1)
        sc = (low | (top << 4)) - 32
        e = np.arange(256)
        h, j, l = e // 128, (e % 128) // 32, e % 32
        q2 = (qs[:, 32 * h + l] >> (2 * j)) & 3
        hb = (hm[:, l] >> (4 * h + j)) & 1
        q = q2 - 4 * (1 - hb)
        scale = d[:, None] * sc[:, 8 * h + 2 * j + (l >= 16)]
        wmin = np.zeros_like(scale)
    else:
        raise ValueError(qtype)
    return (q.reshape(n, k), scale.reshape(n, k).astype(np.float64),
            wmin.reshape(n, k).astype(np.float64))
