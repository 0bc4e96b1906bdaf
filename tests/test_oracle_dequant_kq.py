"""The oracle's K-quant row dequantisers (dequantize_row_q{3,4,5,6}_K, vendor/ggml-subset/generated/
quants_base.c:80-230; the token embedding of a K-quant model, engine.rs:2251-2256), no GPU.

Pinned against the independent block decoder's exact values d * scale * code - dmin * min (tests/
kquant_blocks.py, written from the format description): (1) with power-of-two block scales every
f32 step is exact, so each element equals the exact value; (2) on random blocks each element is the
exact value rounded once to f32. The fp16 d and dmin times a 6-bit scale or min are exact in f32 and
so are their products with a 3- to 5-bit code, so whether the reference's GCC build contracts
d1 * q - m1 into one fused operation (crates/kernels-sys/build.rs:5-7) changes no element."""
import numpy as np
import pytest

import kquant_blocks as KB
import oracle as O

GGML = {3: 11, 4: 12, 5: 13, 6: 14}


def exact(ty, raw, k):
    out = []
    bb = KB.BYTES[ty]
    for b in range(k // 256):
        d, dmin, q, sc, m = KB.decode_block(ty, raw[b * bb:(b + 1) * bb])
        out.append(d * sc.astype(np.float64) * q - dmin * m.astype(np.float64))
    return np.concatenate(out)


@pytest.mark.parametrize("ty", [3, 4, 5, 6])
def test_power_of_two_scales_are_exact(ty):
    raw = KB.random_blocks(ty, 1, 1024, seed=70 + ty, dw=2.0 ** -7, dmin=2.0 ** -9)[0]
    got = O.dequantize_row_kq(GGML[ty], raw, 1024).astype(np.float64)
    assert np.array_equal(got, exact(ty, raw, 1024))


@pytest.mark.parametrize("ty", [3, 4, 5, 6])
def test_random_blocks_are_the_correctly_rounded_exact_values(ty):
    """the one rounding left is the last operation: every element is the exact value rounded once
    to f32 (Q6_K: the product with its 6-bit code is the rounded step)"""
    raw = KB.random_blocks(ty, 1, 256 * 64, seed=80 + ty)[0]
    got = O.dequantize_row_kq(GGML[ty], raw, 256 * 64)
    assert np.array_equal(got, exact(ty, raw, 256 * 64).astype(np.float32))
