"""Small numpy statement of the GGUF block codes and FISH's int8 activations.

Used by the tests as a second, independently written decoder (loop structure
of quant.cpp's dequantisers, not the oracle's per-element formulas), so that
the oracle's integer decomposition is checked against something other than
itself. Pure numpy; slow; for small inputs only.
"""
from __future__ import annotations

import numpy as np

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 8, 12, 13, 14
BLOCK_ELEMS = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}


def f16(b2) -> float:
    return float(np.frombuffer(bytes(bytearray(b2[:2])), np.float16)[0])


def k4_scales(s12):
    s = [int(v) for v in s12]
    sc, mn = [], []
    for j in range(8):
        if j < 4:
            sc.append(s[j] & 63)
            mn.append(s[j + 4] & 63)
        else:
            sc.append((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4))
            mn.append((s[j + 4] >> 4) | ((s[j] >> 6) << 4))
    return sc, mn


def block_codes(t: int, blk: np.ndarray):
    """Integer codes (element order) and per-element integer scale / min / group of one block."""
    blk = np.asarray(blk, np.uint8).astype(np.int64)
    if t == Q8_0:
        return blk[2:34].astype(np.int8).astype(np.int64), None
    if t == Q4_0:
        q = np.concatenate([blk[2:18] & 15, blk[2:18] >> 4]) - 8
        return q, None
    if t in (Q4_K, Q5_K):
        sc, mn = k4_scales(blk[4:16])
        q = np.zeros(256, np.int64)
        if t == Q4_K:
            qs = blk[16:144]
            for j in range(4):
                q[64 * j:64 * j + 32] = qs[32 * j:32 * j + 32] & 15
                q[64 * j + 32:64 * j + 64] = qs[32 * j:32 * j + 32] >> 4
        else:
            qh, qs = blk[16:48], blk[48:176]
            for j in range(4):
                q[64 * j:64 * j + 32] = (qs[32 * j:32 * j + 32] & 15) + 16 * ((qh >> (2 * j)) & 1)
                q[64 * j + 32:64 * j + 64] = (qs[32 * j:32 * j + 32] >> 4) + 16 * ((qh >> (2 * j + 1)) & 1)
        return q, (np.repeat(sc, 32), np.repeat(mn, 32))
    if t == Q6_K:
        ql, qh, scs = blk[0:128], blk[128:192], blk[192:208].astype(np.uint8).astype(np.int8).astype(np.int64)
        q = np.zeros(256, np.int64)
        s = np.zeros(256, np.int64)
        for n in range(2):
            for l in range(32):
                is_ = l // 16
                b = 128 * n
                q[b + l] = (ql[64 * n + l] & 15) | (((qh[32 * n + l] >> 0) & 3) << 4)
                q[b + l + 32] = (ql[64 * n + l + 32] & 15) | (((qh[32 * n + l] >> 2) & 3) << 4)
                q[b + l + 64] = (ql[64 * n + l] >> 4) | (((qh[32 * n + l] >> 4) & 3) << 4)
                q[b + l + 96] = (ql[64 * n + l + 32] >> 4) | (((qh[32 * n + l] >> 6) & 3) << 4)
                s[b + l] = scs[8 * n + is_ + 0]
                s[b + l + 32] = scs[8 * n + is_ + 2]
                s[b + l + 64] = scs[8 * n + is_ + 4]
                s[b + l + 96] = scs[8 * n + is_ + 6]
        return q - 32, s
    raise ValueError(t)


def block_ints(t: int, row: np.ndarray, acts: np.ndarray, n: int) -> np.ndarray:
    """The integers of FISH's AVX2 kernels per block, by brute force."""
    be, bb = BLOCK_ELEMS[t], BLOCK_BYTES[t]
    out = []
    for b in range(n // be):
        blk = row[b * bb:(b + 1) * bb]
        q, extra = block_codes(t, blk)
        if be == 32:
            a = acts[b * 40:(b + 1) * 40]
            xq = a[8:40].astype(np.int8).astype(np.int64)
            out.append(int(np.dot(q, xq)))
        else:
            a = acts[b * 276:(b + 1) * 276]
            xq = a[20:276].astype(np.int8).astype(np.int64)
            if t == Q6_K:
                out.append(int(np.dot(q * extra, xq)))
            else:
                sc, mn = extra
                bs = a[4:20].view(np.int16).astype(np.int64)
                out.append(int(np.dot(q * sc, xq)))
                out.append(int(np.dot(mn[::32], bs)))
    return np.array(out, np.int64)


def dot_from_ints(t: int, row: np.ndarray, acts: np.ndarray, n: int, ints: np.ndarray) -> float:
    """Rebuild the f32-scaled dot from per-block integers (f64 sum)."""
    be, bb = BLOCK_ELEMS[t], BLOCK_BYTES[t]
    total = 0.0
    k = 0
    for b in range(n // be):
        blk = row[b * bb:(b + 1) * bb]
        if be == 32:
            xd = float(acts[b * 40:b * 40 + 4].view(np.float32)[0])
            total += f16(blk[0:2]) * xd * ints[k]
            k += 1
        else:
            xd = float(acts[b * 276:b * 276 + 4].view(np.float32)[0])
            if t == Q6_K:
                total += f16(blk[208:210]) * xd * ints[k]
                k += 1
            else:
                total += f16(blk[0:2]) * xd * ints[k] - f16(blk[2:4]) * xd * ints[k + 1]
                k += 2
    return total


def quantize_acts(x: np.ndarray, block: int) -> np.ndarray:
    """Q8Act (block 32) or Q8ActK (block 256) bytes from the closed form."""
    x = np.asarray(x, np.float32).reshape(-1, block)
    amax = np.max(np.abs(x), axis=1).astype(np.float32)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d > 0, np.float32(1.0) / np.where(d > 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    q = np.clip(np.rint((x * idv[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    out = []
    for i in range(x.shape[0]):
        if block == 32:
            out.append(np.frombuffer(np.float32(d[i]).tobytes() + np.int32(q[i].astype(np.int64).sum()).tobytes()
                                     + q[i].tobytes(), np.uint8))
        else:
            sums = q[i].astype(np.int64).reshape(8, 32).sum(axis=1).astype(np.int16)
            out.append(np.frombuffer(np.float32(d[i]).tobytes() + sums.tobytes() + q[i].tobytes(), np.uint8))
    return np.concatenate(out)
