"""The oracle's K-quant restatement (oracle/kquants.cpp), pinned on the CPU.

quantize_row_q8_K (quants_base.c:14-48): known answers worked out by hand (round half to even,
first maximum, sign of d, zero blocks). Lane GEMVs (oxe_vl_q{3,4,5,6}k.inc): (1) in exact arithmetic
(power-of-two scales, small codes) the result must be the exact dot product of the values an
independent decoder of the ggml block formats (tests/kquant_blocks.py) reads; this pins every bit
field, nibble, scale / min pairing, offset (-32, -4) and sign; (2) on full-range random blocks the
result must equal, bit for bit, the reference's documented float chain evaluated here from that
decoder's integers with exact rationals rounded once per operation (fused where the reference uses
vfmaq_f32, separately rounded where it uses vmlaq_f32 / vmlsq_f32 or a plain multiply), which pins
which operations are fused and their order. The reference holds no stored vectors for these
kernels (its check compares against ggml at run time, crates/kernels-sys/src/tests.rs)."""
from fractions import Fraction

import numpy as np
import pytest

import kquant_blocks as KB
import oracle as O


def q8k(y):
    return np.frombuffer(np.ascontiguousarray(y).tobytes(), KB.Q8K)


# ---- quantize_row_q8_K

def test_q8_K_zero_block():
    y = q8k(O.quantize_q8_K(np.zeros(256, np.float32)))
    assert y["d"][0] == 0 and not y["qs"].any() and not y["bsums"].any()


def test_q8_K_round_half_even_with_unit_scale():
    # the first |max| is -127: iscale = -127 / -127 = 1 exactly, d = 1, codes = round-half-even(x)
    x = np.zeros(256, np.float32)
    x[0] = -127.0
    vals = {1: 2.5, 2: 3.5, 3: -2.5, 4: -0.5, 5: 0.5, 6: 1.5, 7: 126.5, 8: 100.49, 9: -3.5, 10: 127.0}
    for i, v in vals.items():
        x[i] = v
    y = q8k(O.quantize_q8_K(x))
    want = {0: -127, 1: 2, 2: 4, 3: -2, 4: 0, 5: 0, 6: 2, 7: 126, 8: 100, 9: -4, 10: 127}
    for i, q in want.items():
        assert y["qs"][0][i] == q, i
    assert y["d"][0] == 1.0
    assert list(y["bsums"][0][:1]) == [sum(want[i] for i in range(11))]
    assert not y["bsums"][0][1:].any()


def test_q8_K_first_maximum_and_sign():
    # |x| ties at 5: the first (+5) is the max, iscale = -127/5 < 0: codes are negated, d < 0
    x = np.zeros(512, np.float32)
    x[2], x[4] = 5.0, -5.0
    x[300] = -1.0     # second block: its max is -1, iscale = 127, d = 1/127
    y = q8k(O.quantize_q8_K(x))
    assert y["qs"][0][2] == -127 and y["qs"][0][4] == 127
    assert y["d"][0] == np.float32(1) / (np.float32(-127) / np.float32(5)) and y["d"][0] < 0
    assert y["qs"][1][300 - 256] == -127 and y["d"][1] == np.float32(1) / np.float32(127)
    # bsums: sums of 16 codes
    assert y["bsums"][0][0] == 0 and y["bsums"][1][(300 - 256) // 16] == -127


def test_q8_K_bsums_are_sums_of_16():
    x = np.random.default_rng(3).standard_normal((3, 768)).astype(np.float32)
    y = q8k(O.quantize_q8_K(x).reshape(-1))
    assert np.array_equal(y["bsums"].astype(np.int64), y["qs"].reshape(-1, 16, 16).astype(np.int64).sum(-1))
    assert np.abs(y["qs"]).max() == 127


# ---- lane GEMVs in exact arithmetic

@pytest.mark.parametrize("ty", [3, 4, 5, 6])
@pytest.mark.parametrize("dw,dmin,dx", [(1.0, 1.0, 1.0), (2.0 ** -6, 2.0 ** -5, 0.25)])
def test_vl_gemv_exact_cases(ty, dw, dmin, dx):
    k, nr, nl = 512, 5, 3
    w = KB.random_blocks(ty, nr, k, seed=ty, dw=dw, dmin=dmin, scale_lim=40)
    y = KB.q8k_blocks(nl, k, seed=10 + ty, lim=10, d=dx)
    s = O.vl_gemv(ty, w, k, y)
    for l in range(nl):
        for r in range(nr):
            ex = KB.exact_row_dot(ty, w[r], y[l], k)
            assert Fraction(float(s[l, r])) == ex, (l, r)


# ---- lane GEMVs: the documented float chain, exact rationals rounded once per operation

def rnd(v):
    """v (Fraction) rounded to the nearest float32, ties to even (normal range)"""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = 0
    while a >= 2:
        a /= 2
        e += 1
    while a < 1:
        a *= 2
        e -= 1
    m = a * (1 << 23)
    f = m.numerator // m.denominator
    rem = m - f
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and f % 2 == 1):
        f += 1
    return sign * Fraction(f, 1 << 23) * (Fraction(2) ** e)


def chain(ty, wrow, yrow, k):
    y = q8k(yrow)
    bb = KB.BYTES[ty]
    acc = Fraction(0)
    for b in range(k // 256):
        d, dmin, q, sc, m = KB.decode_block(ty, wrow[b * bb:(b + 1) * bb])
        x = y["qs"][b].astype(np.int64)
        dx = Fraction(float(y["d"][b]))
        sub = [int((q[16 * i:16 * i + 16] * x[16 * i:16 * i + 16]).sum()) for i in range(16)]
        bs32 = [int(x[32 * j:32 * j + 32].sum()) for j in range(8)]
        if ty in (4, 5):
            sbs, sbm = rnd(Fraction(d) * dx), rnd(Fraction(dmin) * dx)
            bias_blk = 0
            for sb in range(4):
                for j in (2 * sb, 2 * sb + 1):          # fused: acc = fma(sbs, f32(sc * I), acc)
                    I = sub[2 * j] + sub[2 * j + 1]
                    acc = rnd(sbs * rnd(Fraction(int(sc[32 * j]) * I)) + acc)
                bias = sum(int(m[32 * j]) * bs32[j] for j in (2 * sb, 2 * sb + 1))
                if ty == 5:                              # per step, unfused
                    acc = rnd(acc - rnd(sbm * bias))
                bias_blk += bias
            if ty == 4:                                  # once per block, unfused
                acc = rnd(acc - rnd(Fraction(bias_blk) * sbm))
        elif ty == 6:
            I = sum(int(sc[16 * i]) * sub[i] for i in range(16))
            acc = rnd(acc + rnd(rnd(Fraction(I)) * rnd(Fraction(d) * dx)))      # unfused
        else:
            isum = sum(int(sc[16 * i]) * sub[i] for i in range(16))
            acc = rnd(rnd(Fraction(isum)) * rnd(dx * Fraction(d)) + acc)       # fused
    return acc


@pytest.mark.parametrize("ty", [3, 4, 5, 6])
def test_vl_gemv_float_chain(ty):
    k, nr, nl = 512, 3, 2
    w = KB.random_blocks(ty, nr, k, seed=100 + ty)
    y = O.quantize_q8_K(np.random.default_rng(200 + ty).standard_normal((nl, k)).astype(np.float32) * 3)
    s = O.vl_gemv(ty, w, k, y)
    for l in range(nl):
        for r in range(nr):
            assert Fraction(float(s[l, r])) == chain(ty, w[r], y[l], k), (l, r)


def test_vl_gemv_unknown_type():
    with pytest.raises(ValueError):
        O.vl_gemv(2, np.zeros((1, 84), np.uint8), 256, np.zeros((1, 292), np.uint8))
