"""Pins of the CPU oracle's kernel-level functions (no GPU).

Each check is chosen so that a plausible mistake in the restatement fails it: hand-derived known
answers for the float orders (reduction trees, fp16 accumulation, rounding modes), exact rational
arithmetic for single-rounding operations, independent library routines (numpy's fp16 conversion,
float64 math) with stated tolerances, and brute force on tiny inputs.
The reference holds no numeric vectors for this path (its kernel tests compare two in-tree
implementations on seeded random data, crates/kernels-sys/src/tests.rs:4-46), so the pins are these.
"""
import ctypes as C
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

L = O.lib()
B24 = float(2 ** 24)


# ---- exact rounding of rationals to binary formats (independent of the oracle) ----------------
def round_binary(fr, p, emin, emax):
    """Round a Fraction to the nearest binary float with p significand bits (ties to even)."""
    if fr == 0:
        return 0.0
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, emin)
    scale = Fraction(2) ** (p - 1 - e)
    m = a * scale
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    v = Fraction(n) / scale
    if v > (2 - Fraction(2) ** (1 - p)) * Fraction(2) ** emax:
        return sign * math.inf
    return sign * float(v)


def to_f16(fr):
    return round_binary(fr, 11, -14, 15)


def to_f32(fr):
    return round_binary(fr, 24, -126, 127)


def h2f(h):
    return float(np.array([h], np.uint16).view(np.float16)[0])


def f2h_bits(v):
    return int(np.array([v], np.float16).view(np.uint16)[0])


def fp(a):
    return O.ptr(a, C.c_float)


# ---- fp16 conversions -------------------------------------------------------------------------
def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([L.oxo_f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)
    edges = np.array([65504.0, 65519.99, 65520.0, 2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25, 1 + 2.0 ** -11,
                      1 + 3 * 2.0 ** -11, -(1 + 2.0 ** -11), 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 0.0, -0.0,
                      np.inf, -np.inf], np.float32)
    xs = np.concatenate([bits.view(np.float32), edges])
    xs = xs[~np.isnan(xs)]
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([L.oxo_f32_to_f16(float(v)) for v in xs], np.uint16)
    assert np.array_equal(got, ref)
    # hand-derived ties: 1 + 2^-11 is halfway between 1 and 1 + 2^-10 -> even (1.0)
    assert L.oxo_f32_to_f16(1 + 2.0 ** -11) == 0x3C00
    assert L.oxo_f32_to_f16(1 + 3 * 2.0 ** -11) == 0x3C02
    assert L.oxo_f32_to_f16(65520.0) == 0x7C00


# ---- fp16 FMA: one rounding (vfmaq_f16), checked with exact rationals ------------------------
def test_f16_fma_single_rounding():
    rng = np.random.default_rng(1)
    cases = []
    for _ in range(3000):
        a, b, c = (int(v) for v in rng.integers(0, 0x7C00, 3))
        sa, sb, sc = (int(v) << 15 for v in rng.integers(0, 2, 3))
        cases.append((a | sa, b | sb, c | sc))
    # cancellation: c close to -a*b, where rounding the product first changes the result
    for _ in range(2000):
        a, b = (int(v) for v in rng.integers(0x2000, 0x5800, 2))
        pr = h2f(a) * h2f(b)
        c = f2h_bits(-pr) ^ int(rng.integers(0, 4))
        cases.append((a, b, c))
    for a, b, c in cases:
        exact = Fraction(h2f(a)) * Fraction(h2f(b)) + Fraction(h2f(c))
        want = to_f16(exact)
        got = h2f(L.oxo_f16_fma(a, b, c))
        if want == 0:
            assert got == 0, (hex(a), hex(b), hex(c))
        else:
            assert got == want, (hex(a), hex(b), hex(c), got, want)
    # hand case: (1+2^-10)^2 - 1 = 2^-9 + 2^-20 exactly -> fp16 (ulp 2^-19 at 2^-9): tie -> 2^-9
    one_p = 0x3C01
    assert h2f(L.oxo_f16_fma(one_p, one_p, 0xBC00)) == 2.0 ** -9


# ---- Q8_0 activation quantizer (quants_subset.c:6-42) -----------------------------------------
def quant(x):
    return O.quantize_q8_0(np.asarray(x, np.float32))


def test_quantize_zero_block():
    q, d = quant(np.zeros(64, np.float32))
    assert not q.any() and not d.any()


def test_quantize_round_half_even_codes():
    x = np.zeros(32, np.float32)
    x[:8] = [127.0, -64.5, 0.5, 1.5, 2.5, -0.5, -2.5, 126.5]
    q, d = quant(x)
    # amax 127 -> d = 1, id = 1; codes are round-half-even of x (vcvtnq_s32_f32)
    assert d[0] == 0x3C00
    assert list(q[:8]) == [127, -64, 0, 2, 2, 0, -2, 126]


def test_quantize_negative_amax():
    x = np.zeros(32, np.float32)
    x[:3] = [-254.0, 3.0, 5.0]
    q, d = quant(x)
    assert d[0] == 0x4000          # d = 254/127 = 2
    assert list(q[:3]) == [-127, 2, 2]   # 1.5 -> 2, 2.5 -> 2 (ties to even)


def test_quantize_uses_f32_inverse_scale():
    # amax 1: x * 127 = 2.49993.. -> 2 with id = 1/d from the f32 d; the fp16-rounded d would give 3
    x = np.zeros(32, np.float32)
    x[0], x[1] = 1.0, 0.019684476777911186
    q, d = quant(x)
    assert q[1] == 2
    assert d[0] == np.float32(1.0 / 127).astype(np.float16).view(np.uint16)


def test_quantize_properties_random():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((16, 2048)) * rng.uniform(1e-3, 1e3, (16, 1))).astype(np.float32)
    q, d = quant(x)
    xb = x.reshape(16, 64, 32)
    qb = q.reshape(16, 64, 32).astype(np.int32)
    amax_idx = np.abs(xb).argmax(-1)
    # the element of largest magnitude maps to +-127
    assert np.all(np.abs(np.take_along_axis(qb, amax_idx[..., None], -1)) == 127)
    d32 = (np.abs(xb).max(-1) / np.float32(127)).astype(np.float32)
    # codes within half a step of x / d (f32 scale)
    assert np.all(np.abs(xb / d32[..., None] - qb) <= 0.5 + 1e-4)
    assert np.array_equal(d, d32.astype(np.float16).view(np.uint16))


def test_dequantize():
    q = np.arange(-16, 16, dtype=np.int8)
    d = np.array([0x3800], np.uint16)   # 0.5
    y = np.empty(32, np.float32)
    L.oxo_dequantize_row_q8_0(O.ptr(q, C.c_int8), O.ptr(d, C.c_uint16), 32, fp(y))
    assert np.array_equal(y, q.astype(np.float32) * 0.5)


# ---- Q8_0 GEMV: exact integers + fp32 FMA chain from +0 (repack_subset.cpp:1633-1679) --------
def test_gemv_bruteforce_exact():
    rng = np.random.default_rng(3)
    k, nr, nl = 128, 6, 2
    wq = rng.integers(-127, 128, (nr, k)).astype(np.int8)
    wq[0, :32] = -127           # extreme blocks, as the reference's bitwise tests use
    wq[1, 32:64] = 127
    wd = np.float32(rng.uniform(0.001, 0.021, (nr, k // 32))).astype(np.float16).view(np.uint16)
    x = rng.standard_normal((nl, k)).astype(np.float32)
    x[1, :32] = 127.0
    xq, xd = O.quantize_q8_0(x)
    y, isum = O.gemv_q8_0(wq, wd, xq, xd, want_isum=True)
    for l in range(nl):
        for r in range(nr):
            acc = 0.0
            for b in range(k // 32):
                s = int(np.dot(wq[r, 32 * b:32 * b + 32].astype(np.int64), xq[l, 32 * b:32 * b + 32].astype(np.int64)))
                assert isum[l, r, b] == s
                prod = to_f32(Fraction(h2f(xd[l, b])) * Fraction(h2f(wd[r, b])))
                acc = to_f32(Fraction(s) * Fraction(prod) + Fraction(acc))
            assert np.float32(acc) == y[l, r], (l, r, acc, y[l, r])


def test_gemv_row_range_equals_full():
    wq, wd, x, xq, xd = O.config1_inputs(0)
    wq, wd = wq[:256], wd[:256]
    full = O.gemv_q8_0(wq, wd, xq, xd)
    part = O.gemv_q8_0(wq[64:192], wd[64:192], xq, xd)
    assert np.array_equal(full[:, 64:192], part)
    one = O.gemv_q8_0(wq, wd, xq[1:], xd[1:])
    assert np.array_equal(full[1:], one)


# ---- ggml_vec_dot_f32 order (vec.cpp:104-125, simd-mappings.h:358-395) ------------------------
def dot32(p):
    x = np.asarray(p, np.float32)
    y = np.ones_like(x)
    return L.oxo_vec_dot_f32(len(x), fp(x), fp(y))


def prods(n, nz):
    p = np.zeros(n, np.float32)
    for i, v in nz.items():
        p[i] = v
    return p


def test_vec_dot_f32_reduction_tree():
    # element i of a 16-step goes to lane i%4 of accumulator (i%16)//4; a0+=a2, a1+=a3, a0+=a1;
    # then (l0+l1)+(l2+l3). Each case separates the reference order from one plausible other order.
    # lane 3: a0 = 1, a1 = 2^24 + 2 (exact), a0 + a1 = 2^24 + 3 -> tie -> 2^24 + 4
    # ((acc0+acc1)+(acc2+acc3) would give 2^24 + 2)
    assert dot32(prods(16, {3: 1, 7: B24, 15: 2})) == B24 + 4
    # lanes: r1 = 2, r2 = 1, r3 = 2^24: (r0+r1)+(r2+r3) = 2 + 2^24 (1 + 2^24 rounds to 2^24)
    # (a sequential lane sum would give 2^24 + 4)
    assert dot32(prods(16, {3: B24, 5: 2, 10: 1})) == B24 + 2
    # r0 = 2^24, r2 = 1, r3 = 1: (r0+r1)+(r2+r3) = 2^24 + 2 ((r0+r2)+(r1+r3) would give 2^24)
    assert dot32(prods(16, {3: 1, 4: B24, 10: 1})) == B24 + 2
    # r0 = 2^24, r1 = 2, r3 = 1: (2^24 + 2) + 1 -> tie -> 2^24 + 4 (element order: 2^24 + 2)
    assert dot32(prods(16, {4: B24, 7: 1, 9: 2})) == B24 + 4
    # elements i and i+16 share a chain: 2^24 + 1 + 1 in one fma chain stays 2^24
    assert dot32(prods(48, {0: B24, 16: 1, 32: 1})) == B24


def test_vec_dot_f32_random_close_to_exact():
    rng = np.random.default_rng(4)
    for n in (16, 128, 2048):
        x = rng.standard_normal(n).astype(np.float32)
        y = rng.standard_normal(n).astype(np.float32)
        exact = float(np.dot(x.astype(np.float64), y.astype(np.float64)))
        got = L.oxo_vec_dot_f32(n, fp(x), fp(y))
        assert abs(got - exact) <= 1e-5 * float(np.abs(x).dot(np.abs(y)))


# ---- ggml_vec_dot_f16 (vec.cpp:345-371, simd-mappings.h:400-429) ------------------------------
def test_vec_dot_f16_fp16_accumulators():
    # 32 fp16 chains each add 1.0 2100 times: fp16 stops at 2048 (2049 ties to even); the reduce
    # adds chains in fp16 (4096, 8192), widens, and sums 4 x 16384 in f32 -> 65536, not 67200.
    n = 32 * 2100
    one = np.full(n, 0x3C00, np.uint16)
    assert L.oxo_vec_dot_f16(n, O.ptr(one, C.c_uint16), O.ptr(one, C.c_uint16)) == 65536.0
    # leftovers after the last full 32-step are added in double
    x = np.full(35, 0x3C00, np.uint16)
    assert L.oxo_vec_dot_f16(35, O.ptr(x, C.c_uint16), O.ptr(x, C.c_uint16)) == 35.0


def test_vec_dot_f16_random_close():
    rng = np.random.default_rng(5)
    for n in (64, 256, 1000):
        x = rng.standard_normal(n).astype(np.float16)
        y = (rng.standard_normal(n) * 0.1).astype(np.float16)
        exact = float(np.dot(x.astype(np.float64), y.astype(np.float64)))
        got = L.oxo_vec_dot_f16(n, O.ptr(x.view(np.uint16), C.c_uint16), O.ptr(y.view(np.uint16), C.c_uint16))
        assert abs(got - exact) <= 2e-3 * float(np.abs(x.astype(np.float64)).dot(np.abs(y.astype(np.float64))))


# ---- ggml_v_expf / silu / swiglu / softmax (vec.h:1154-1185, vec.cpp:380-440, 625-697) -------
def test_v_expf_accuracy():
    xs = np.concatenate([np.linspace(-87.0, 88.0, 20001), [0.0, 1.0, -1.0, 1e-8, -1e-8]]).astype(np.float32)
    for x in xs:
        got = L.oxo_v_expf(float(x))
        want = math.exp(float(x))
        ulp = np.spacing(np.float32(want))
        assert abs(got - want) <= 2 * float(ulp), (x, got, want)
    assert L.oxo_v_expf(0.0) == 1.0
    # deep underflow and overflow branches
    assert L.oxo_v_expf(-150.0) == 0.0
    assert L.oxo_v_expf(100.0) == math.inf
    assert abs(L.oxo_v_expf(-100.0) - math.exp(-100.0)) <= 2 * 2.0 ** -149


def test_silu_swiglu():
    rng = np.random.default_rng(6)
    n = 1027                      # a tail after the groups of 4
    x = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    y = np.empty(n, np.float32)
    L.oxo_silu_f32(n, fp(y), fp(x))
    want = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    assert np.allclose(y, want, rtol=4e-7, atol=1e-30)
    L.oxo_swiglu_f32(n, fp(y), fp(x), fp(u))
    assert np.allclose(y, want * u, rtol=1e-6, atol=1e-30)


def test_soft_max():
    rng = np.random.default_rng(7)
    n = 300
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    mask = np.zeros(n, np.float32)
    mask[250:] = -np.inf
    y = np.empty(n, np.float32)
    w = np.empty(n, np.float32)
    L.oxo_soft_max_f32(n, fp(y), fp(x), np.float32(0.0625), fp(mask), fp(w))
    z = x[:250].astype(np.float64) * 0.0625
    want = np.exp(z - z.max())
    want /= want.sum()
    assert np.all(y[250:] == 0.0)
    assert np.allclose(y[:250], want, rtol=2e-6, atol=0)
    assert abs(float(y.astype(np.float64).sum()) - 1.0) < 1e-5


# ---- top-k (oxe_ops.cpp:121-165) -------------------------------------------------------------
def topk(x, k):
    x = np.asarray(x, np.float32)
    out = np.empty(k, np.int32)
    scratch = np.empty(len(x), np.int32)
    tie = C.c_int(-1)
    L.oxo_argsort_top_k_f32(fp(x), len(x), k, O.ptr(out, C.c_int32), O.ptr(scratch, C.c_int32), C.byref(tie))
    return list(out), tie.value


def test_topk_distinct():
    rng = np.random.default_rng(8)
    for _ in range(50):
        x = rng.permutation(256).astype(np.float32) * np.float32(0.01) - 1
        ids, tie = topk(x, 8)
        assert ids == list(np.argsort(-x, kind="stable")[:8]) and tie == 0


def test_topk_ties_flagged():
    x = np.zeros(256, np.float32)
    x[[5, 9, 17]] = [3.0, 2.0, 2.0]
    x[[40, 41, 42, 43, 44, 45]] = 1.0
    ids, tie = topk(x, 8)
    assert tie == 1
    assert ids[0] == 5 and sorted(ids[1:3]) == [9, 17] and set(ids[3:]) <= {40, 41, 42, 43, 44, 45}
    # the 9th value equal to the 8th also counts as a tie (the selection would be ambiguous)
    x = np.arange(256, dtype=np.float32)
    x[100] = x[247]
    _, tie = topk(x, 8)
    assert tie == 1


# ---- norms (oxe_ops.cpp:19-49) -----------------------------------------------------------------
def test_rms_norm_mul():
    rng = np.random.default_rng(9)
    eps = np.float32(1e-6)
    for scale in (1.0, 1e-3):     # at 1e-3 the mean square is 1e-6, comparable to eps
        x = (rng.standard_normal(2048) * scale).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
        y = np.empty_like(x)
        L.oxo_rms_norm_mul_f32(fp(x), fp(w), fp(y), 2048, eps)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w
        assert np.allclose(y, want, rtol=1e-6, atol=0)


def test_gdn_l2_norm():
    rng = np.random.default_rng(10)
    for scale in (1.0, 1e-4):
        x = (rng.standard_normal(128) * scale).astype(np.float32)
        y = x.copy()
        L.oxo_gdn_l2_norm_f32(fp(y), 128, np.float32(1e-6))
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt(np.sum(x64 * x64) + 1e-6)
        assert np.allclose(y, want, rtol=2e-6, atol=0)


# ---- conv step (oxe_ops.cpp:175-201) -----------------------------------------------------------
def test_conv_step_exact_and_order():
    nr, nc = 3, 4
    state = np.array([[1, 2, 3], [0, 0, 0], [B24, 0, 0]], np.float32)
    c = np.array([[1, 1, 1, 1], [2, -1, 3, 5], [1, 1, 1, 1]], np.float32)
    x_new = np.array([4, 7, 1], np.float32)
    x_new[2] = 0
    state[2] = [B24, 1, 1]
    out = np.empty(nr, np.float32)
    L.oxo_ssm_conv_step_f32(fp(state), fp(x_new), fp(c), nr, nc, fp(out))
    assert out[0] == 10.0 and out[1] == 35.0
    # products added in order: 2^24 + 1 -> 2^24, + 1 -> 2^24 (a pairwise sum would give 2^24 + 2)
    assert out[2] == B24
    # the window shifts by one: the new input becomes the last state entry
    assert list(state[0]) == [2, 3, 4] and list(state[1]) == [0, 0, 7]


# ---- gated delta rule (oxe_ops.cpp:207-251, 268-345) ------------------------------------------
def dn_step(s, q, k, v, g, beta):
    sv = len(q)
    so = np.empty_like(s)
    out = np.empty(sv, np.float32)
    L.oxo_gated_delta_net_step_f32_from(fp(so), fp(s), fp(q), fp(k), fp(v), np.float32(g), np.float32(beta), sv, fp(out))
    return so, out


def test_delta_rule_math():
    rng = np.random.default_rng(11)
    sv = 128
    s = (rng.standard_normal((sv, sv)) * 0.1).astype(np.float32)   # row j = column j of S
    q, k, v = (rng.standard_normal(sv).astype(np.float32) for _ in range(3))
    k /= np.float32(np.linalg.norm(k))
    g, beta = -0.3, 0.7
    so, out = dn_step(s, q, k, v, g, beta)
    S = s.astype(np.float64).T * math.exp(g)          # S[i][j]
    kk, qq, vv = (a.astype(np.float64) for a in (k, q, v))
    delta = (vv - S.T @ kk) * beta
    S = S + np.outer(kk, delta)
    want_out = (S.T @ qq) / math.sqrt(sv)
    assert np.allclose(so.T, S, rtol=1e-5, atol=1e-6)
    assert np.allclose(out, want_out, rtol=1e-4, atol=1e-5)


def test_delta_rule_update_is_fused():
    """The rank-1 update row += k * delta is one fused multiply-add per element (ggml_vec_mad_f32's
    vfmaq_f32, oxe_ops.cpp:324), not a rounded product then a sum. Hand-derived case: S = 0 but
    S[0][0] = -1, k = e0 * (1 + 2^-12), v = 0, beta = 1, g = 0 (decay 1). Then sk = -(1 + 2^-12) and
    delta = 1 + 2^-12 exactly; the fused update gives (1 + 2^-12)^2 - 1 = 2^-11 + 2^-24 exactly,
    where the unfused one rounds the product to 1 + 2^-11 (a tie, to even) and gives 2^-11."""
    sv = 16
    s = np.zeros((sv, sv), np.float32)
    s[0, 0] = -1.0
    k = np.zeros(sv, np.float32)
    k[0] = np.float32(1.0 + 2.0 ** -12)
    q = np.zeros(sv, np.float32)
    q[0] = 1.0
    v = np.zeros(sv, np.float32)
    so, out = dn_step(s, q, k, v, 0.0, 1.0)
    fused = np.float32(2.0 ** -11 + 2.0 ** -24)
    assert so[0, 0] == fused, (so[0, 0], fused, np.float32(2.0 ** -11))
    assert np.array_equal(so[1:], s[1:]) and np.array_equal(so[0, 1:], s[0, 1:])
    assert out[0] == fused / np.float32(4.0) and not out[1:].any()


def test_delta_rule_special_cases():
    rng = np.random.default_rng(12)
    sv = 16
    s = rng.standard_normal((sv, sv)).astype(np.float32)
    q, k, v = (rng.standard_normal(sv).astype(np.float32) for _ in range(3))
    # g = 0, beta = 0: the state is unchanged and out = S^T q / 4
    so, out = dn_step(s, q, k, v, 0.0, 0.0)
    assert np.array_equal(so, s)
    # k = 0: only the decay acts
    so, _ = dn_step(s, q, np.zeros(sv, np.float32), v, -1.0, 0.5)
    assert np.array_equal(so, s * np.float32(math.exp(-1.0)))


# ---- RoPE (oxe_ops.cpp:386-455) ----------------------------------------------------------------
def rope_cache(p):
    cache = np.empty(64, np.float32)
    sec = np.array([11, 11, 10, 0], np.int32)
    L.oxo_mrope_cache_init(p, O.ptr(sec, C.c_int32), 1, 64, 64, np.float32(1e7), 1.0, 0.0, 1.0, 32.0, 1.0,
                           262144, 0, fp(cache))
    return cache


def test_rope_cache_and_rotation():
    c0 = rope_cache(0)
    assert np.all(c0[0::2] == 1.0) and np.all(c0[1::2] == 0.0)
    x = np.random.default_rng(13).standard_normal(256).astype(np.float32)
    y = x.copy()
    L.oxo_rope_neox_inplace(fp(y), 64, fp(c0))
    assert np.array_equal(x, y)                       # position 0 is the identity
    p = 517
    c = rope_cache(p)
    theta = p * (1e7 ** (-np.arange(32) * 2 / 64.0))   # text positions: all IMRoPE sections share p
    assert np.allclose(c[0::2], np.cos(theta), atol=2e-4)
    assert np.allclose(c[1::2], np.sin(theta), atol=2e-4)
    y = x.copy()
    L.oxo_rope_neox_inplace(fp(y), 64, fp(c))
    x0, x1 = x[:32].astype(np.float64), x[32:64].astype(np.float64)
    cc, ss = c[0::2].astype(np.float64), c[1::2].astype(np.float64)
    assert np.allclose(y[:32], x0 * cc - x1 * ss, atol=1e-6)
    assert np.allclose(y[32:64], x0 * ss + x1 * cc, atol=1e-6)
    assert np.array_equal(y[64:], x[64:])             # only the first n_rot dims rotate


# ---- attention head (oxe_ops.cpp:465-493) -----------------------------------------------------
def test_attention_head():
    rng = np.random.default_rng(14)
    hd, n_kv, pos = 256, 512, 300
    q = rng.standard_normal(hd).astype(np.float32)
    kc = (rng.standard_normal((n_kv, hd)) * 0.2).astype(np.float16)
    k_last = (rng.standard_normal(hd) * 0.2).astype(np.float16)
    vt = rng.standard_normal((hd, n_kv + 32)).astype(np.float16)
    out = np.empty(hd, np.float32)

    def run(kc, vt, k_last):
        L.oxo_attn_head_f16(fp(q), O.ptr(kc.view(np.uint16), C.c_uint16), hd, O.ptr(k_last.view(np.uint16), C.c_uint16),
                            O.ptr(vt.view(np.uint16), C.c_uint16), n_kv + 32, n_kv, pos, hd, np.float32(1 / 16), fp(out))
        return out.copy()

    o1 = run(kc, vt, k_last)
    # float64 attention with the reference's fp16 formats: q and the probabilities rounded to fp16,
    # both dot products accumulated in fp16 chains (f64_model.dot_f16, the NEON ggml_vec_dot_f16
    # structure pinned bit for bit by test_vec_dot_f16_reduce_tree_separating)
    from f64_model import dot_f16, f16
    keys = kc[:n_kv].astype(np.float64).copy()
    keys[pos] = k_last
    sc = dot_f16(keys[: pos + 1], f16(q)) / 16
    p = np.exp(sc - sc.max())
    p16 = np.zeros(n_kv)
    p16[: pos + 1] = f16(p / p.sum())
    want = dot_f16(vt[:, :n_kv].astype(np.float64), p16)
    assert np.abs(o1 - want).max() <= 1e-3 * np.abs(want).max()
    # an exact-math reference (no fp16 accumulation) is further away than the bar: the fp16 chains matter
    exact = vt[:, : pos + 1].astype(np.float64) @ (p / p.sum())
    assert np.abs(exact - want).max() > np.abs(o1 - want).max()
    # masked positions and the cache's own row at pos_last do not matter
    kc2, vt2 = kc.copy(), vt.copy()
    kc2[pos:] = 7
    vt2[:, pos + 1:] = 3
    assert np.array_equal(run(kc2, vt2, k_last), o1)


# ---- bit-separating cases for the double-precision sums and the fp16 reduce tree ---------------
# Each expected value is derived with exact rationals rounded once per operation in the reference's
# structure; each case is chosen so that a plausible other structure gives different bits (asserted).
def to_f64(fr):
    return round_binary(fr, 53, -1022, 1023)


def rms_ref(x, w, eps, square="f32", acc="f64"):
    """oxe_rms_norm_mul_f32 (oxe_ops.cpp:32-42): sum += (double)(x*x) in element order; mean = f32(sum / n);
    scale = 1 / sqrtf(mean + eps); y = (x * scale) * w. `square` / `acc` select plausible other forms."""
    s = Fraction(0)
    for v in x:
        sq = Fraction(float(v)) ** 2
        sq = Fraction(to_f32(sq)) if square == "f32" else sq
        s = Fraction(to_f32(s + sq)) if acc == "f32" else Fraction(to_f64(s + sq))
    mean = np.float32(to_f32(s / len(x)))
    scale = np.float32(1.0) / np.sqrt(np.float32(mean + np.float32(eps)))   # f32 ops, correctly rounded
    return (x * scale) * w


def rms_oracle(x, w, eps):
    y = np.empty_like(x)
    L.oxo_rms_norm_mul_f32(fp(x), fp(w), fp(y), len(x), np.float32(eps))
    return y


def test_rms_norm_double_sum_separating():
    eps = np.float32(1e-6)
    # (1) one large square and 2047 squares of 2^-26: a double sum keeps them (mean 2^-11 (1 + 2047 2^-26)),
    # an f32 sum loses every one of them (mean 2^-11)
    x = np.full(2048, 2.0 ** -13, np.float32)
    x[0] = 1.0
    w = np.ones(2048, np.float32)
    want = rms_ref(x, w, eps)
    assert not np.array_equal(want, rms_ref(x, w, eps, acc="f32"))
    assert np.array_equal(rms_oracle(x, w, eps).view(np.uint32), want.view(np.uint32))
    # (2) squares rounded to f32 before the double sum: a seeded search for a row on which the
    # unrounded (double) squares give other bits
    rng = np.random.default_rng(31)
    for _ in range(200):
        x = (1 + rng.integers(0, 2 ** 12, 256) * 2.0 ** -12 + rng.integers(0, 2, 256) * 2.0 ** -23).astype(np.float32)
        w = np.ones(256, np.float32)
        want = rms_ref(x, w, eps)
        if not np.array_equal(want, rms_ref(x, w, eps, square="f64")):
            break
    else:
        raise AssertionError("no separating row found")
    assert np.array_equal(rms_oracle(x, w, eps).view(np.uint32), want.view(np.uint32))


def softmax_ref(x, e, group="pairwise", acc="f64"):
    """oxe_soft_max_f32 with scale 1 and no mask over n % 4 == 0 values whose exponentials are e
    (ggml_vec_soft_max_f32, NEON: per group of 4, sum += (double)vaddvq_f32(e0..e3); then
    y = e * f32(1.0 / sum))."""
    s = Fraction(0)
    for g in range(0, len(e), 4):
        a = [Fraction(float(v)) for v in e[g:g + 4]]
        if group == "pairwise":
            gs = to_f32(Fraction(to_f32(a[0] + a[1])) + Fraction(to_f32(a[2] + a[3])))
        elif group == "sequential":
            gs = to_f32(Fraction(to_f32(Fraction(to_f32(a[0] + a[1])) + a[2])) + a[3])
        else:                                   # the group added to the double sum element by element
            for v in a:
                s = Fraction(to_f64(s + v))
            continue
        s = Fraction(to_f32(s + Fraction(gs))) if acc == "f32" else Fraction(to_f64(s + Fraction(gs)))
    r = np.float32(to_f32(Fraction(to_f64(1 / s))))
    return np.asarray(e, np.float32) * r


def test_soft_max_group_sums_separating():
    n = 256
    x = np.full(n, -20.5, np.float32)
    x[0] = 0.0                                  # the maximum: e = 1
    x[1:4] = -16.54                             # e ~ 1.1 * 2^-24: the group's add order decides its last bit
    # the tail (e ~ 1e-9 each, lost in an f32 sum next to 1) shifts 1 / sum; the first tail value on
    # which every other structure gives other bits is taken
    for tail in np.arange(-21.0, -19.0, 0.05, dtype=np.float32):
        x[4:] = tail
        e = np.array([L.oxo_v_expf(float(v)) for v in x], np.float32)
        want = softmax_ref(x, e)
        if all(not np.array_equal(want, softmax_ref(x, e, **o))
               for o in (dict(group="sequential"), dict(group="none"), dict(acc="f32"))):
            break
    else:
        raise AssertionError("no separating tail found")
    y = np.empty(n, np.float32)
    w = np.empty(n, np.float32)
    L.oxo_soft_max_f32(n, fp(y), fp(x), np.float32(1.0), None, fp(w))
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def f16x8_reduce_ref(chains, tree="ref"):
    """GGML_F16x8_REDUCE (simd-mappings.h:410-428) over accumulators a0..a3 of 8 fp16 lanes:
    a0 += a2, a1 += a3, a0 += a1 (fp16 adds per lane); t = f32(lanes 0-3) + f32(lanes 4-7);
    vaddvq: (t0 + t1) + (t2 + t3)."""
    a = [[Fraction(float(v)) for v in chains[8 * j:8 * j + 8]] for j in range(4)]
    add16 = lambda p, q: [Fraction(to_f16(u + v)) for u, v in zip(p, q)]
    if tree == "ref":
        a0 = add16(add16(a[0], a[2]), add16(a[1], a[3]))
    elif tree == "sequential":
        a0 = add16(add16(add16(a[0], a[1]), a[2]), a[3])
    else:                                       # "adjacent": (a0 + a1) + (a2 + a3)
        a0 = add16(add16(a[0], a[1]), add16(a[2], a[3]))
    if tree == "lanes_adjacent":
        a0 = add16(add16(a[0], a[2]), add16(a[1], a[3]))
        t = [Fraction(to_f32(a0[2 * i] + a0[2 * i + 1])) for i in range(4)]
    else:
        t = [Fraction(to_f32(a0[i] + a0[i + 4])) for i in range(4)]
    if tree == "lanes_sequential":
        return to_f32(Fraction(to_f32(Fraction(to_f32(t[0] + t[1])) + t[2])) + t[3])
    return to_f32(Fraction(to_f32(t[0] + t[1])) + Fraction(to_f32(t[2] + t[3])))


def test_vec_dot_f16_reduce_tree_separating():
    # n = 32 with y = 1: chain c (accumulator c // 8, lane c % 8) holds exactly x_c. The chain values
    # are drawn (seeded) from values whose fp16 and f32 sums round, until every other tree gives
    # other bits.
    rng = np.random.default_rng(37)
    pool = np.array([0, 0, 0, 1, 1, 2, 3, 2048, 2048, 1024, 2.0 ** -13, 2.0 ** -12, 0.5], np.float64)
    for _ in range(5000):
        c = rng.choice(pool, 32).astype(np.float16)
        want = f16x8_reduce_ref(c)
        if all(f16x8_reduce_ref(c, o) != want for o in ("sequential", "adjacent", "lanes_adjacent", "lanes_sequential")):
            break
    else:
        raise AssertionError("no separating chain values found")
    one = np.ones(32, np.float16)
    got = L.oxo_vec_dot_f16(32, O.ptr(c.view(np.uint16), C.c_uint16), O.ptr(one.view(np.uint16), C.c_uint16))
    assert got == want
