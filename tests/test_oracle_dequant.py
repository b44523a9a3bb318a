"""CPU: block dequantization (Q8_0, Q4_K, Q2_K, F16, BF16) pinned by hand-built blocks.

Expected values come from the format definitions (ggml-common.h:252-338; Q8_0 and Q4_K value
formulas in dequant.hpp:80-86,157-190; Q2_K from ggml's dequantize_row_q2_K, which the
reference does not vendor) with the scale/min codes chosen by the test, plus literal anchors
worked out by hand; every value is rounded once from the exact product to F16.
"""
import numpy as np
import pytest


def f16(x):
    return np.float16(x).view(np.uint16)


def test_q8_0_known_block(orc):
    q = np.array([-128, -1, 0, 1, 127, 2, -2, 64] + list(range(-12, 12)), np.int8)
    blk = np.concatenate([np.uint16([0x3800]).view(np.uint8), q.view(np.uint8)])  # d = 0.5
    got = orc.dequant(1, blk, 32)
    assert list(got[:8]) == [f16(-64), f16(-0.5), 0x0000, f16(0.5), f16(63.5), f16(1.0), f16(-1.0), f16(32.0)]
    assert np.array_equal(got, (q.astype(np.float64) * 0.5).astype(np.float16).view(np.uint16))
    neg = blk.copy()
    neg[:2] = np.uint16([0xB400]).view(np.uint8)  # d = -0.25: a zero code decodes to -0.0
    gotn = orc.dequant(1, neg, 32)
    assert gotn[2] == 0x8000 and gotn[0] == f16(32.0)


def _q4k_block():
    sc = [1, 2, 3, 4, 37, 50, 63, 17]
    mn = [5, 6, 7, 8, 20, 33, 47, 60]
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    qs = ((np.arange(128) * 7 + 3) & 0xFF).astype(np.uint8)
    blk = np.concatenate([np.uint16([0x3C00, 0x3800]).view(np.uint8), s, qs])  # d = 1, dmin = 0.5
    return blk, sc, mn, qs


def test_q4_k_known_block(orc):
    blk, sc, mn, qs = _q4k_block()
    assert blk.size == 144
    got = orc.dequant(2, blk, 256).view(np.float16).astype(np.float64)
    # literal anchors (element: value)
    assert got[0] == 0.5 and got[32] == -3.0 and got[200] == 669.5 and got[255] == 89.0
    exp = np.empty(256)
    for e in range(256):
        g, w = divmod(e, 64)
        byte = qs[32 * g + (w % 32)]
        q = (byte & 0xF) if w < 32 else (byte >> 4)
        pair = 2 * g + (w >= 32)
        exp[e] = 1.0 * sc[pair] * q - 0.5 * mn[pair]
    assert np.array_equal(got, exp.astype(np.float16).astype(np.float64))


def test_q2_k_known_block(orc):
    scales = np.array([(i % 16) | ((15 - i) << 4) for i in range(16)], np.uint8)
    qs = ((np.arange(64) * 37 + 11) & 0xFF).astype(np.uint8)
    blk = np.concatenate([scales, qs, np.uint16([0x3800, 0x3400]).view(np.uint8)])  # d = 0.5, dmin = 0.25
    assert blk.size == 84
    got = orc.dequant(3, blk, 256).view(np.float16).astype(np.float64)
    assert got[0] == -3.75 and got[100] == 3.75 and got[255] == 0.0
    exp = np.empty(256)
    for e in range(256):
        n, r = divmod(e, 128)
        j, w = divmod(r, 32)
        q = (qs[32 * n + w] >> (2 * j)) & 3
        s = scales[e // 16]
        exp[e] = 0.5 * (s & 0xF) * q - 0.25 * (s >> 4)
    assert np.array_equal(got, exp.astype(np.float16).astype(np.float64))


def test_f16_bf16_rows(orc):
    x = np.random.default_rng(0).standard_normal(512).astype(np.float32) * 3
    h = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.dequant(4, h.view(np.uint8), 512), h)
    b = (x.view(np.uint32) >> 16).astype(np.uint16)  # truncated BF16 values
    want = (b.astype(np.uint32) << 16).view(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.dequant(5, b.view(np.uint8), 512), want)


@pytest.mark.parametrize("fmt,tol", [(1, 0.01), (2, 0.12), (3, 0.45)])
def test_quantizer_round_trip(moe, orc, fmt, tol):
    """The product's quantizer writes valid blocks: dequantized values track the input."""
    rows, k = 8, 1024
    x = moe.synth_normal_f32(3, fmt, 0.02, rows * k)
    q = moe.quantize(fmt, x, rows, k)
    assert q.size == rows * orc.lib().or_row_bytes(fmt, k)
    y = orc.dequant(fmt, q, rows * k).view(np.float16).astype(np.float64)
    rel = np.sqrt(np.mean((y - x) ** 2) / np.mean(x.astype(np.float64) ** 2))
    assert rel < tol, rel


def test_row_bytes(moe, orc):
    for fmt, k, b in [(1, 2048, 2176), (2, 2048, 1152), (3, 4096, 1344), (4, 512, 1024), (5, 512, 1024)]:
        assert orc.lib().or_row_bytes(fmt, k) == b == moe.row_bytes(fmt, k)
    assert moe.row_bytes(2, 300) == 0 and moe.row_bytes(1, 48) == 0
