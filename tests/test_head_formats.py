"""Pins of the oracle's speech_head weight formats (oracle/cbx_oracle.cpp):
ggml's Q4_0 / Q5_0 / Q8_0 blocks of 32 (fp16 scale d first; Q4_0 element
j < 16 in the low nibble of byte j, element j + 16 in its high nibble,
w = (q - 8) d; Q5_0 a little-endian 32-bit word qh after d whose bit j is the
fifth bit of element j, then nibbles as Q4_0, w = (q - 16) d; Q8_0 w = q d),
quantized with the rules the reference's converter gets from
gguf.quants.quantize (scripts/convert-t3-turbo-to-gguf.py:78-104; Q4_0 / Q5_0:
d = the signed largest-magnitude value / -8 or / -16, q = trunc(x / d + 8.5
or 16.5) clipped to [0, 15] or [0, 31]; Q8_0: d = max|x| / 127, q = round
half away from zero).  Known-answer blocks worked by hand, the error bounds
the rules imply on random rows, and the binary64 head against a direct
product.  gguf-py itself is not installed here: the quantizer (which only
makes test weights; the kernels read whatever blocks a file holds) is pinned
by the hand-worked blocks alone.
"""
import numpy as np

import oracle_lib as O


def test_q4_0_known_block():
    # x_j = (j - 16) / 4: the largest magnitude is x_0 = -4, so d = 0.5 and
    # q_j = trunc(j / 2 + 0.5) = 0,1,1,2,2,...,15,15, with 16 clipped to 15
    x = ((np.arange(32) - 16) / 4.0).astype(np.float32)[None, :]
    b = O.quantize(x, O.WTYPE_Q4_0)[0]
    want = bytes([0x00, 0x38,  # d = 0.5 in binary16
                  0x80, 0x91, 0x91, 0xA2, 0xA2, 0xB3, 0xB3, 0xC4,
                  0xC4, 0xD5, 0xD5, 0xE6, 0xE6, 0xF7, 0xF7, 0xF8])
    assert bytes(b) == want
    q = [0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 5, 6, 6, 7, 7, 8,
         8, 9, 9, 10, 10, 11, 11, 12, 12, 13, 13, 14, 14, 15, 15, 15]
    deq = O.dequantize(b[None, :], O.WTYPE_Q4_0, 32)[0]
    assert list(deq) == [(v - 8) * 0.5 for v in q]


def test_q8_0_known_blocks():
    # |x| <= 127 integers with 127 present: d = 1 and q = x; halved: d = 0.5
    x = np.array([-127, -100, -64, -3, -1, 0, 1, 2, 5, 9, 17, 33, 50, 63, 64, 65,
                  70, 80, 90, 99, 101, 110, 111, 112, 113, 120, 121, 122, 123, 124, 126, 127],
                 np.float32)
    rows = np.stack([x, x / 2]).astype(np.float32)
    b = O.quantize(rows, O.WTYPE_Q8_0)
    assert bytes(b[0][:2]) == bytes([0x00, 0x3C])  # d = 1.0
    assert bytes(b[1][:2]) == bytes([0x00, 0x38])  # d = 0.5
    assert list(b[0][2:].view(np.int8)) == list(x.astype(np.int8))
    assert list(b[1][2:].view(np.int8)) == list(x.astype(np.int8))
    deq = O.dequantize(b, O.WTYPE_Q8_0, 32)
    assert np.array_equal(deq, rows)


def test_q5_0_known_block():
    # x_j = (p_j - 16) / 2 for a permutation p of 0..31 (p_1 = 0: the largest
    # magnitude is x_1 = -8, so d = 0.5 and q_j = trunc(p_j + 0.5) = p_j).
    # qs byte j = (p_j & 15) | (p_{j+16} & 15) << 4; qh bit j = p_j >> 4.
    p = [25, 0, 17, 8, 30, 3, 12, 21, 6, 29, 14, 1, 19, 10, 27, 4,
         11, 22, 2, 31, 16, 7, 24, 13, 9, 28, 5, 18, 15, 26, 20, 23]
    x = ((np.array(p) - 16) / 2.0).astype(np.float32)[None, :]
    b = O.quantize(x, O.WTYPE_Q5_0)[0]
    want = bytes([0x00, 0x38,              # d = 0.5 in binary16
                  0x95, 0x52, 0x5A, 0xEA,  # qh, little-endian
                  0xB9, 0x60, 0x21, 0xF8, 0x0E, 0x73, 0x8C, 0xD5,
                  0x96, 0xCD, 0x5E, 0x21, 0xF3, 0xAA, 0x4B, 0x74])
    assert bytes(b) == want
    deq = O.dequantize(b[None, :], O.WTYPE_Q5_0, 32)[0]
    assert np.array_equal(deq, x[0])  # every step of 0.5 in [-8, 7.5] is exact


def test_q5_0_clipped_block():
    # the largest magnitude positive (x_0 = 8): d = -0.5; -8 maps to
    # trunc(32.5) = 32, clipped to 31 (-7.5); 0.25 -> 16, -0.25 -> 17,
    # 0.3 -> trunc(15.9) = 15, -0.3 -> 17, 7.7 -> 1, -7.74 -> 31, 0 -> 16
    x = np.zeros(32, np.float32)
    x[:8] = [8, -8, 0.25, -0.25, 0.3, -0.3, 7.7, -7.74]
    b = O.quantize(x[None, :], O.WTYPE_Q5_0)[0]
    want = bytes([0x00, 0xB8,              # d = -0.5
                  0xAE, 0xFF, 0xFF, 0xFF,  # fifth bits: q = 0,31,16,17,15,17,1,31, then 16s
                  0x00, 0x0F, 0x00, 0x01, 0x0F, 0x01, 0x01, 0x0F] + [0x00] * 8)
    assert bytes(b) == want
    deq = O.dequantize(b[None, :], O.WTYPE_Q5_0, 32)[0]
    assert list(deq[:8]) == [8.0, -7.5, 0.0, -0.5, 0.5, -0.5, 7.5, -7.5]
    assert np.all(deq[8:] == 0.0)


def test_q5_0_dequant_of_planted_bits():
    # each of the 32 elements in turn: q = 16 + 15 (only its fifth bit and
    # all four nibble bits set) against q = 16 elsewhere, d = 1 -- a wrong
    # qh bit order, nibble half or offset moves the value off its element
    for j in range(32):
        blk = np.zeros(22, np.uint8)
        blk[0:2] = [0x00, 0x3C]            # d = 1.0
        qh = 0xFFFFFFFF                    # every element's fifth bit: q >= 16
        blk[2:6] = np.frombuffer(qh.to_bytes(4, "little"), np.uint8)
        blk[6 + (j % 16)] = 0x0F if j < 16 else 0xF0
        deq = O.dequantize(blk[None, :], O.WTYPE_Q5_0, 32)[0]
        want = np.zeros(32, np.float32)
        want[j] = 15.0
        assert np.array_equal(deq, want), j
    blk = np.zeros(22, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    assert np.all(O.dequantize(blk[None, :], O.WTYPE_Q5_0, 32)[0] == -16.0)  # q = 0


def _scales(blocks, wtype, n_embd):
    bb = O.BLOCK_BYTES[wtype]
    nb = n_embd // 32
    raw = blocks.reshape(blocks.shape[0], nb, bb)[:, :, :2].copy()
    return raw.view(np.float16)[..., 0].astype(np.float32)


def test_quantize_error_bounds():
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((64, 256)) * 0.05).astype(np.float32)
    w[3, :32] = 0.0  # an all-zero block: d = 0, every weight 0
    for wtype, frac, qmax in ((O.WTYPE_Q4_0, 1.0, 8), (O.WTYPE_Q5_0, 1.0, 16),
                              (O.WTYPE_Q8_0, 0.5, 127)):
        b = O.quantize(w, wtype)
        assert b.shape == (64, 256 // 32 * O.BLOCK_BYTES[wtype])
        d = np.abs(_scales(b, wtype, 256))
        deq = O.dequantize(b, wtype, 256)
        err = np.abs(deq - w).reshape(64, 8, 32).max(axis=-1)
        # Q4_0 / Q5_0 round to the nearest step except the clipped top step (one d);
        # Q8_0 to the nearest step; the binary16 scale (quantization divides
        # by the binary32 one) moves a weight q d by up to |q| d 2^-11
        assert np.all(err <= d * (frac + (qmax + 1) * 2.0 ** -11) + 1e-12)
        assert np.all(deq[3, :32] == 0.0)
        # the largest-magnitude weight of each Q4_0 / Q5_0 block is exact (q = 0)
        if wtype in (O.WTYPE_Q4_0, O.WTYPE_Q5_0):
            blk = w.reshape(64, 8, 32)
            i = np.abs(blk).argmax(axis=-1)
            mx = np.take_along_axis(blk, i[..., None], -1)[..., 0]
            dq = np.take_along_axis(deq.reshape(64, 8, 32), i[..., None], -1)[..., 0]
            assert np.allclose(dq, mx, rtol=2.0 ** -10, atol=0)


def test_head_f64_matches_direct_product():
    rng = np.random.default_rng(12)
    V, K, R = 37, 64, 3
    w = (rng.standard_normal((V, K)) * 0.1).astype(np.float32)
    h = rng.standard_normal((R, K)).astype(np.float32)
    bias = rng.standard_normal(V).astype(np.float32)
    for wtype in (O.WTYPE_Q4_0, O.WTYPE_Q5_0, O.WTYPE_Q8_0, O.WTYPE_F16):
        b = O.quantize(w, wtype)
        got = O.head_f64(b, wtype, bias, h, V, K)
        deq = O.dequantize(b, wtype, K).astype(np.float64)
        want = h.astype(np.float64) @ deq.T + bias.astype(np.float64)
        assert np.allclose(got, want, rtol=1e-13, atol=1e-13)


def _split_rows(x):
    """The matrix-core head's activation split, restated in numpy: each row
    scaled by 2^s (s = 14 - E for a largest magnitude in [2^E, 2^(E+1)),
    clamped to [-126, 126]; 0 for a zero row), then hi = fp16(y) and
    lo = fp16(y - hi) with y = x * 2^s, each rounded to nearest."""
    x = np.asarray(x, np.float32)
    mx = np.max(np.abs(x), axis=1)
    e = np.frexp(np.where(mx > 0, mx, 1.0))[1].astype(np.int64) - 1
    s = np.where(mx > 0, np.clip(14 - e, -126, 126), 0)
    sc = np.ldexp(np.float32(1.0), s).astype(np.float32)[:, None]
    y = (x * sc).astype(np.float32)
    hi = y.astype(np.float16)
    lo = (y - hi.astype(np.float32)).astype(np.float16)
    return y, hi, lo


def test_fp16_split_bound():
    """|x 2^s - hi - lo| <= 2^-23 |x 2^s| + 2^-25 on rows of every magnitude
    fp32 holds (subnormal 1e-40 .. 3e38, far past the fp16 range either way),
    and no part overflows: the bound the head's error budget rests on.  Rows
    above 2^-112 land in [2^14, 2^15); smaller ones take the largest scale."""
    rng = np.random.default_rng(11)
    rows = []
    for mag in (1e-40, 1e-30, 1e-8, 1e-3, 1.0, 3e4, 1e6, 1e30, 1e35):
        r = (rng.standard_normal((4, 1024)) * mag).astype(np.float32)
        r[0, ::7] = 0.0
        r[1, 5] = np.float32(mag * 1e3)  # one entry far above the rest
        rows.append(r)
    top = np.full((2, 1024), 1.0, np.float32)
    top[:, 3] = np.finfo(np.float32).max  # the largest finite float
    top[1, 4] = -np.finfo(np.float32).max
    rows.append(top)
    x = np.concatenate(rows)
    assert np.all(np.isfinite(x))
    y, hi, lo = _split_rows(x)
    assert np.all(np.isfinite(hi)) and np.all(np.isfinite(lo))
    err = np.abs(y.astype(np.float64) - hi.astype(np.float64) - lo.astype(np.float64))
    bound = 2.0 ** -23 * np.abs(y.astype(np.float64)) + 2.0 ** -25
    assert np.all(err <= bound)
    mx = np.max(np.abs(x), axis=1)
    m = np.max(np.abs(y), axis=1)
    big = mx >= 2.0 ** -112
    assert np.all((m[big] >= 2.0 ** 14) & (m[big] < 2.0 ** 15))
    assert np.array_equal(y[~big], (x[~big] * np.float32(2.0 ** 126)).astype(np.float32))
    assert big.sum() >= 30 and (~big).sum() >= 4


def test_fp16_integer_weights():
    """The head's integer weights in fp16: a byte b placed under the exponent
    of 1024 is 1024 + b exactly, and one fp16 subtraction leaves the Q4_0
    value n - 8 (b = n <= 15) or the Q8_0 value q (b = q ^ 0x80), exactly."""
    b = np.arange(256, dtype=np.uint16)
    f = (np.uint16(0x6400) | b).view(np.float16)
    assert np.array_equal(f.astype(np.float64), 1024.0 + b)
    n = b[:16]
    q4 = (f[:16] - np.float16(1032.0)).astype(np.float64)
    assert np.array_equal(q4, n.astype(np.float64) - 8)
    q = np.arange(-128, 128)
    u = (q.astype(np.int64) & 0xFF) ^ 0x80
    q8 = (f[u] - np.float16(1152.0)).astype(np.float64)
    assert np.array_equal(q8, q.astype(np.float64))
