"""K-quant test data: random ggml blocks (Q3_K, Q4_K, Q5_K, Q6_K) and q8_K activation blocks, and an
independent decoder of the block formats (ggml-common.h:315-376; the element layout of ggml's
dequantize_row_q*_K) into exact integers: value of element e = d * sc(e) * q(e) - dmin * m(e).
Written from the format description element by element, not from the oracle's loops."""
import numpy as np

QK = 256
BYTES = {3: 110, 4: 144, 5: 176, 6: 210}
Q8K = np.dtype([("d", "<f4"), ("qs", "i1", (QK,)), ("bsums", "<i2", (16,))])


def f16_bits(v):
    return np.asarray(v, np.float16).view(np.uint16)


def random_blocks(ty, rows, k, seed, d_range=(1e-3, 1e-2), dw=None, dmin=None, scale_lim=None):
    """rows x k/256 random blocks: random code and scale bytes, fp16 d (and dmin) drawn from d_range
    or fixed (dw / dmin); scale_lim bounds the Q6_K int8 scales (exact-arithmetic tests)"""
    rng = np.random.default_rng(seed)
    nb = k // QK
    b = rng.integers(0, 256, size=(rows, nb, BYTES[ty]), dtype=np.uint8)

    def put_f16(off, fixed):
        v = rng.uniform(*d_range, size=(rows, nb)) if fixed is None else np.full((rows, nb), fixed)
        h = f16_bits(v)
        b[:, :, off] = h & 0xFF
        b[:, :, off + 1] = h >> 8

    if ty in (4, 5):
        put_f16(0, dw)
        put_f16(2, dmin)
    elif ty == 6:
        put_f16(208, dw)
        if scale_lim is not None:
            b[:, :, 192:208] = rng.integers(-scale_lim, scale_lim + 1, size=(rows, nb, 16)).astype(np.int8).view(np.uint8)
    elif ty == 3:
        put_f16(108, dw)
    return b.reshape(rows, nb * BYTES[ty])


def q8k_blocks(nl, k, seed, lim=127, d=None):
    """activation blocks with random codes in [-lim, lim], consistent bsums, d random or fixed"""
    rng = np.random.default_rng(seed)
    nb = k // QK
    y = np.zeros((nl, nb), Q8K)
    y["qs"] = rng.integers(-lim, lim + 1, size=(nl, nb, QK))
    y["bsums"] = y["qs"].reshape(nl, nb, 16, 16).astype(np.int32).sum(-1)
    y["d"] = rng.uniform(-0.05, 0.05, size=(nl, nb)) if d is None else d
    return y.view(np.uint8).reshape(nl, nb * 292)


def _u16(blk, off):
    return int(blk[off]) | int(blk[off + 1]) << 8


def _f16(blk, off):
    return float(np.uint16(_u16(blk, off)).view(np.float16))


def _k4_scales(sc12):
    """the eight 6-bit (scale, min) pairs of a Q4_K / Q5_K block: scales j < 4 in the low 6 bits of
    bytes j (mins: j + 4); j >= 4 from the nibbles of bytes j + 4 and the top 2 bits of bytes j - 4
    (scales) and j (mins)"""
    out = []
    for j in range(8):
        if j < 4:
            out.append((sc12[j] & 63, sc12[j + 4] & 63))
        else:
            out.append(((sc12[j + 4] & 15) | ((sc12[j - 4] >> 6) << 4), (sc12[j + 4] >> 4) | ((sc12[j] >> 6) << 4)))
    return out


def _q3_scales(sc12):
    """the sixteen 6-bit Q3_K scales: low 4 bits from the nibbles of bytes 0..7 (scale i < 8: low
    nibble of byte i, i >= 8: high nibble of byte i - 8), high 2 bits from bytes 8..11 (scale i:
    bits 2 (i // 4) of byte 8 + i % 4)"""
    out = []
    for i in range(16):
        lo = (sc12[i] & 15) if i < 8 else (sc12[i - 8] >> 4)
        hi = (sc12[8 + i % 4] >> (2 * (i // 4))) & 3
        out.append(lo | hi << 4)
    return out


def decode_block(ty, blk):
    """(d, dmin, q[256], sc[256], m[256]): exact integer codes and per-element scale / min factors"""
    blk = [int(v) for v in blk]
    q = np.zeros(QK, np.int64)
    sc = np.zeros(QK, np.int64)
    m = np.zeros(QK, np.int64)
    if ty in (4, 5):
        d, dmin = _f16(blk, 0), _f16(blk, 2)
        pairs = _k4_scales(blk[4:16])
        qs = blk[16:144] if ty == 4 else blk[48:176]
        qh = blk[16:48] if ty == 5 else None
        for e in range(QK):
            g, r = divmod(e, 64)            # 64-weight group, position inside it
            half, l = divmod(r, 32)         # low nibbles: first 32, high nibbles: next 32
            byte = qs[32 * g + l]
            v = (byte >> 4) if half else (byte & 15)
            if ty == 5:
                v |= ((qh[l] >> (2 * g + half)) & 1) << 4
            q[e] = v
            sc[e], m[e] = pairs[2 * g + half]
        return d, dmin, q, sc, m
    if ty == 6:
        ql, qh, s8 = blk[0:128], blk[128:192], np.array(blk[192:208], np.uint8).view(np.int8)
        d = _f16(blk, 208)
        for e in range(QK):
            n, r = divmod(e, 128)
            quarter, l = divmod(r, 32)
            lb = ql[64 * n + l + (32 if quarter in (1, 3) else 0)]
            low4 = (lb >> 4) if quarter >= 2 else (lb & 15)
            high2 = (qh[32 * n + l] >> (2 * quarter)) & 3
            q[e] = (low4 | high2 << 4) - 32
            sc[e] = int(s8[e // 16])
        return d, 0.0, q, sc, m
    if ty == 3:
        hm, qs = blk[0:32], blk[32:96]
        raw = _q3_scales(blk[96:108])
        d = _f16(blk, 108)
        for e in range(QK):
            n, r = divmod(e, 128)
            s, l = divmod(r, 32)
            low2 = (qs[32 * n + l] >> (2 * s)) & 3
            hbit = (hm[l] >> (4 * n + s)) & 1
            q[e] = low2 - (0 if hbit else 4)
            sc[e] = raw[e // 16] - 32
        return d, 0.0, q, sc, m
    raise ValueError(ty)


def exact_row_dot(ty, wrow, yrow, k):
    """sum over blocks of d_w d_x (sum sc q x) - dmin_w d_x (sum m x), in exact rationals (float64 of
    exact integers times the block's d values; exact when every d is a power of two)"""
    from fractions import Fraction
    nb = k // QK
    bb = BYTES[ty]
    y = np.frombuffer(np.ascontiguousarray(yrow).tobytes(), Q8K)
    tot = Fraction(0)
    for b in range(nb):
        d, dmin, q, sc, m = decode_block(ty, wrow[b * bb:(b + 1) * bb])
        x = y["qs"][b].astype(np.int64)
        dx = Fraction(float(y["d"][b]))
        tot += Fraction(d) * dx * int((sc * q * x).sum()) - Fraction(dmin) * dx * int((m * x).sum())
    return tot
