"""Independent numpy decoders of the ggml block formats, used to pin the C oracle.

Written per element from the block layouts (element index -> the bytes/bits that encode it),
not as a transcription of the oracle's loops, so an index or operand slip in either one shows up
as a mismatch. f32 arithmetic keeps the reference's operation order (e.g. (d*sc)*q - dmin*m) so
the comparison is bit-exact. Sign bits come from the closed form ksigns(i) = i | parity(i) << 7
and never from a table.
"""
import numpy as np

f32 = np.float32


def _h(blk, off):
    return blk[:, off:off + 2].copy().view(np.float16).astype(np.float32).reshape(-1)


def _u32(blk, off):
    return blk[:, off:off + 4].copy().view("<u4").reshape(-1).astype(np.uint64)


def ksigns_closed(i):
    i = np.asarray(i, dtype=np.uint64)
    par = np.zeros_like(i)
    for b in range(7):
        par ^= (i >> np.uint64(b)) & np.uint64(1)
    return i | (par << np.uint64(7))


def _elem_index():
    return np.arange(256)


def q8_0(raw):
    blk = raw.reshape(-1, 34)
    d = _h(blk, 0)[:, None]
    q = blk[:, 2:34].view(np.int8).astype(np.float32)
    return (q * d).astype(np.float32).reshape(-1)


def _scale_min(sc12, j):
    """6-bit (scale, min) of sub-block j (0..7) from the 12 packed bytes, per block."""
    s = sc12.astype(np.int64)
    if j < 4:
        return s[:, j] & 63, s[:, j + 4] & 63
    return (s[:, j + 4] & 15) | ((s[:, j - 4] >> 6) << 4), (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)


def q4_k(raw):
    blk = raw.reshape(-1, 144)
    nb = blk.shape[0]
    d, dmin = _h(blk, 0), _h(blk, 2)
    out = np.empty((nb, 256), dtype=np.float32)
    for i in range(256):
        j = i // 32            # sub-block of 32
        l = i % 32
        byte = blk[:, 16 + 32 * (j // 2) + l].astype(np.int64)
        q = (byte & 15) if j % 2 == 0 else (byte >> 4)
        sc, mn = _scale_min(blk[:, 4:16], j)
        out[:, i] = (d * sc.astype(f32)) * q.astype(f32) - dmin * mn.astype(f32)
    return out.reshape(-1)


def q5_k(raw):
    blk = raw.reshape(-1, 176)
    nb = blk.shape[0]
    d, dmin = _h(blk, 0), _h(blk, 2)
    out = np.empty((nb, 256), dtype=np.float32)
    for i in range(256):
        j, l = i // 32, i % 32
        byte = blk[:, 48 + 32 * (j // 2) + l].astype(np.int64)
        lo = (byte & 15) if j % 2 == 0 else (byte >> 4)
        hi = (blk[:, 16 + l].astype(np.int64) >> j) & 1
        sc, mn = _scale_min(blk[:, 4:16], j)
        out[:, i] = (d * sc.astype(f32)) * (lo + 16 * hi).astype(f32) - dmin * mn.astype(f32)
    return out.reshape(-1)


def q6_k(raw):
    blk = raw.reshape(-1, 210)
    nb = blk.shape[0]
    d = _h(blk, 208)
    out = np.empty((nb, 256), dtype=np.float32)
    for i in range(256):
        half, r = i // 128, i % 128
        quarter, l = r // 32, r % 32
        ql = blk[:, 64 * half + l + 32 * (quarter % 2)].astype(np.int64)
        nib = (ql >> 4) if quarter >= 2 else (ql & 15)
        qh = (blk[:, 128 + 32 * half + l].astype(np.int64) >> (2 * quarter)) & 3
        q = (nib | (qh << 4)) - 32
        sc = blk[:, 192 + 8 * half + l // 16 + 2 * quarter].view(np.int8).astype(f32)
        out[:, i] = (d * sc) * q.astype(f32)
    return out.reshape(-1)


def q2_k(raw):
    blk = raw.reshape(-1, 84)
    nb = blk.shape[0]
    d, dmin = _h(blk, 80), _h(blk, 82)
    out = np.empty((nb, 256), dtype=np.float32)
    for i in range(256):
        half, r = i // 128, i % 128
        shift_j, r2 = r // 32, r % 32
        part, l = r2 // 16, r2 % 16
        sc = blk[:, 8 * half + 2 * shift_j + part].astype(np.int64)
        q = (blk[:, 16 + 32 * half + 16 * part + l].astype(np.int64) >> (2 * shift_j)) & 3
        out[:, i] = (d * (sc & 15).astype(f32)) * q.astype(f32) - dmin * (sc >> 4).astype(f32)
    return out.reshape(-1)


def q3_k(raw):
    blk = raw.reshape(-1, 110)
    nb = blk.shape[0]
    d = _h(blk, 108)
    sraw = blk[:, 96:108].astype(np.int64)
    out = np.empty((nb, 256), dtype=np.float32)
    for i in range(256):
        half, r = i // 128, i % 128
        j, r2 = r // 32, r % 32
        part, l = r2 // 16, r2 % 16
        s_idx = 8 * half + 2 * j + part                      # 0..15
        low = (sraw[:, s_idx] & 15) if s_idx < 8 else (sraw[:, s_idx - 8] >> 4)
        high = (sraw[:, 8 + (s_idx % 4)] >> (2 * (s_idx // 4))) & 3
        sc = (low | (high << 4)) - 32
        q = (blk[:, 32 + 32 * half + 16 * part + l].astype(np.int64) >> (2 * j)) & 3
        hbit = (blk[:, 16 * part + l].astype(np.int64) >> (4 * half + j)) & 1
        out[:, i] = (d * sc.astype(f32)) * (q - 4 * (1 - hbit)).astype(f32)
    return out.reshape(-1)


def iq2_xxs(raw, grid):
    blk = raw.reshape(-1, 66)
    nb = blk.shape[0]
    d = _h(blk, 0)
    out = np.empty((nb, 256), dtype=np.float32)
    grid = np.asarray(grid, dtype=np.uint64)
    for ib in range(8):
        a0, a1 = _u32(blk, 2 + 8 * ib), _u32(blk, 6 + 8 * ib)
        db = (d * (f32(0.5) + (a1 >> np.uint64(28)).astype(f32))) * f32(0.25)
        for l in range(4):
            g = grid[(a0 >> np.uint64(8 * l)) & np.uint64(255)]
            s = ksigns_closed((a1 >> np.uint64(7 * l)) & np.uint64(127))
            for j in range(8):
                gv = ((g >> np.uint64(8 * j)) & np.uint64(255)).astype(f32)
                neg = ((s >> np.uint64(j)) & np.uint64(1)).astype(bool)
                out[:, 32 * ib + 8 * l + j] = np.where(neg, -(db * gv), db * gv)
    return out.reshape(-1)


def iq2_s(raw, grid):
    blk = raw.reshape(-1, 82)
    nb = blk.shape[0]
    d = _h(blk, 0)
    out = np.empty((nb, 256), dtype=np.float32)
    grid = np.asarray(grid, dtype=np.uint64)
    for ib in range(8):
        sc = blk[:, 74 + ib].astype(np.int64)
        qh = blk[:, 66 + ib].astype(np.int64)
        for l in range(4):
            s4 = (sc >> (4 * (l // 2))) & 15
            dl = (d * (f32(0.5) + s4.astype(f32))) * f32(0.25)
            idx = blk[:, 2 + 4 * ib + l].astype(np.int64) | (((qh >> (2 * l)) & 3) << 8)
            g = grid[idx]
            s = blk[:, 34 + 4 * ib + l].astype(np.int64)
            for j in range(8):
                gv = ((g >> np.uint64(8 * j)) & np.uint64(255)).astype(f32)
                out[:, 32 * ib + 8 * l + j] = np.where((s >> j) & 1, -(dl * gv), dl * gv)
    return out.reshape(-1)


def iq3_xxs(raw, grid):
    blk = raw.reshape(-1, 98)
    nb = blk.shape[0]
    d = _h(blk, 0)
    out = np.empty((nb, 256), dtype=np.float32)
    grid = np.asarray(grid, dtype=np.uint64)
    for ib in range(8):
        aux = _u32(blk, 66 + 4 * ib)
        db = (d * (f32(0.5) + (aux >> np.uint64(28)).astype(f32))) * f32(0.5)
        for l in range(4):
            s = ksigns_closed((aux >> np.uint64(7 * l)) & np.uint64(127))
            for j in range(8):
                gi = blk[:, 2 + 8 * ib + 2 * l + j // 4]
                gv = ((grid[gi] >> np.uint64(8 * (j % 4))) & np.uint64(255)).astype(f32)
                neg = ((s >> np.uint64(j)) & np.uint64(1)).astype(bool)
                out[:, 32 * ib + 8 * l + j] = np.where(neg, -(db * gv), db * gv)
    return out.reshape(-1)


def iq4_xs(raw, kvalues):
    blk = raw.reshape(-1, 136)
    nb = blk.shape[0]
    d = _h(blk, 0)
    sh = blk[:, 2:4].copy().view("<u2").reshape(-1).astype(np.int64)
    out = np.empty((nb, 256), dtype=np.float32)
    kv = np.asarray(kvalues, dtype=np.int64)
    for i in range(256):
        ib, r = i // 32, i % 32
        ls = ((blk[:, 4 + ib // 2].astype(np.int64) >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
        byte = blk[:, 8 + 16 * ib + (r % 16)].astype(np.int64)
        nib = (byte & 15) if r < 16 else (byte >> 4)
        out[:, i] = (d * (ls - 32).astype(f32)) * kv[nib].astype(f32)
    return out.reshape(-1)
