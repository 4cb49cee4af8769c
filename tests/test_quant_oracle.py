"""Pins of the quantized-row oracle (oracle/hymt_quant.c) on the CPU.

Each format gets an encoder written here from the block description (the
inverse of the reference's DequantizeRow, BlockLayout.cs:9-106), and the
oracle must decode what it encodes: a wrong nibble order, scale unpacking,
lane stride or codebook index breaks the round trip.  Known-value blocks pin
the value positions by hand-computed numbers."""
import numpy as np
import pytest

from oracle import oracle as O

RNG = np.random.default_rng(7)


def f16(x):
    return np.float16(x).view(np.uint16)


def le16(v):
    v = int(v)
    return bytes([v & 0xFF, v >> 8])


# ---- encoders (one block at a time) ---------------------------------------------

def enc_q8_0(x):
    d = np.float16(max(np.abs(x).max(), 1e-8) / 127.0)
    q = np.clip(np.rint(x / np.float32(d)), -128, 127).astype(np.int8)
    return le16(d.view(np.uint16)) + q.tobytes()


def pack_k4_scales(sc, m):
    """12 bytes from six-bit scales sc[8] and mins m[8] (inverse of
    Q4K.GetScaleMin, Q4K.cs:8-19)."""
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4)
    return bytes(s)


def enc_q4_k(d, dmin, sc, m, q):
    """q[256] nibbles by value position: position 64g + l (l < 32) is the low
    nibble of qs[32g + l], position 64g + 32 + l its high nibble."""
    qs = bytearray(128)
    for g in range(4):
        for l in range(32):
            qs[32 * g + l] = (q[64 * g + l] & 0xF) | ((q[64 * g + 32 + l] & 0xF) << 4)
    return le16(f16(d)) + le16(f16(dmin)) + pack_k4_scales(sc, m) + bytes(qs)


def enc_q6_k(d, sc, q):
    """q[256] six-bit codes (value = d sc[pos // 16] (q - 32))."""
    ql, qh = bytearray(128), bytearray(64)
    for h in range(2):
        for l in range(32):
            b = 128 * h
            q1, q2, q3, q4 = q[b + l], q[b + 32 + l], q[b + 64 + l], q[b + 96 + l]
            ql[64 * h + l] = (q1 & 0xF) | ((q3 & 0xF) << 4)
            ql[64 * h + 32 + l] = (q2 & 0xF) | ((q4 & 0xF) << 4)
            qh[32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    return bytes(ql) + bytes(qh) + np.asarray(sc, np.int8).tobytes() + le16(f16(d))


def enc_q2_0c(d, c):
    """c[512] codes 0..3 (value (2c - 3) d), four consecutive codes per byte."""
    qs = bytes(int(c[4 * i] | (c[4 * i + 1] << 2) | (c[4 * i + 2] << 4) | (c[4 * i + 3] << 6)) for i in range(128))
    return le16(f16(d)) + qs


CODEBOOK = [0xA9, 0x89, 0x29, 0x09, 0xA6, 0x86, 0x26, 0x06, 0x9A, 0x92, 0x1A, 0x12, 0x6A, 0x62, 0x4A, 0x42,
            0x01, 0x21, 0x81, 0xA1, 0x04, 0x24, 0x84, 0xA4, 0x10, 0x18, 0x90, 0x98, 0x40, 0x48, 0x60, 0x68]


def enc_stq1_0(d, t):
    """t[256] ternary values whose every group (chunk c, position g of 16:
    lanes at 64c + g + 16 lane) is a codebook pattern (STQ1_0.cs:57-101)."""
    qs, sign = bytearray(32), bytearray(8)
    for grp in range(64):
        chunk, gloc = grp >> 4, grp & 15
        lanes = [int(t[64 * chunk + gloc + 16 * ln]) + 1 for ln in range(4)]
        pat = lanes[0] | (lanes[1] << 2) | (lanes[2] << 4) | (lanes[3] << 6)
        idx = CODEBOOK.index(pat)
        qs[grp >> 1] |= (idx & 0xF) << ((grp & 1) * 4)
        sign[grp >> 3] |= (idx >> 4) << (grp & 7)
    return bytes(qs) + bytes(sign) + le16(f16(d))


# ---- tests ---------------------------------------------------------------------

def test_row_bytes_match_block_layout():
    # BlockLayout.cs:17-31: Q4_K 144, Q6_K 210, Q8_0 34/32, Q2_0C 130/512, STQ1_0 42/256
    assert O.row_bytes(O.W_Q4_K, 2048) == 8 * 144
    assert O.row_bytes(O.W_Q6_K, 2048) == 8 * 210
    assert O.row_bytes(O.W_Q8_0, 2048) == 64 * 34
    assert O.row_bytes(O.W_Q2_0C, 2048) == 4 * 130
    assert O.row_bytes(O.W_STQ1_0, 2048) == 8 * 42


def test_q8_0_round_trip_and_known_block():
    x = RNG.standard_normal(256).astype(np.float32)
    raw = b"".join(enc_q8_0(x[i:i + 32]) for i in range(0, 256, 32))
    y = O.dequant(O.W_Q8_0, raw, 1, 256)[0]
    d = np.abs(x).reshape(8, 32).max(axis=1) / 127
    assert np.all(np.abs(y - x).reshape(8, 32) <= 0.51 * d[:, None] + 1e-3 * np.abs(x).reshape(8, 32))
    blk = le16(0x3800) + np.arange(-16, 16, dtype=np.int8).tobytes()  # d = 0.5
    assert np.array_equal(O.dequant(O.W_Q8_0, blk, 1, 32)[0], 0.5 * np.arange(-16, 16))


def test_q4_k_value_positions():
    # all nibbles 1, scale of sub-block j = j + 1, no mins, d = 1: value = j + 1
    sc, m = list(range(1, 9)), [0] * 8
    y = O.dequant(O.W_Q4_K, enc_q4_k(1.0, 0.0, sc, m, [1] * 256), 1, 256)[0]
    assert np.array_equal(y, np.repeat(np.arange(1, 9), 32).astype(np.float32))


def test_q4_k_round_trip():
    for _ in range(20):
        d, dmin = 2.0 ** RNG.integers(-8, -2), 2.0 ** RNG.integers(-8, -2)
        sc, m = RNG.integers(0, 64, 8), RNG.integers(0, 64, 8)
        q = RNG.integers(0, 16, 256)
        y = O.dequant(O.W_Q4_K, enc_q4_k(d, dmin, sc, m, q), 1, 256)[0]
        sub = np.arange(256) // 32
        assert np.allclose(y, d * sc[sub] * q - dmin * m[sub], rtol=0, atol=1e-6)


def test_q6_k_round_trip():
    for _ in range(20):
        d = 2.0 ** RNG.integers(-10, -4)
        sc = RNG.integers(-128, 128, 16)
        q = RNG.integers(0, 64, 256)
        y = O.dequant(O.W_Q6_K, enc_q6_k(d, sc, q), 1, 256)[0]
        assert np.allclose(y, d * sc[np.arange(256) // 16] * (q - 32), rtol=1e-6, atol=0)


def test_q2_0c_round_trip():
    for _ in range(10):
        d = 2.0 ** RNG.integers(-8, 0)
        c = RNG.integers(0, 4, 512)
        y = O.dequant(O.W_Q2_0C, enc_q2_0c(d, c), 1, 512)[0]
        assert np.array_equal(y, ((2 * c - 3) * d).astype(np.float32))


def test_stq1_0_codebook_and_round_trip():
    # STQ1_0.cs:11-13: every group has one zero and three equal-magnitude lanes
    for pat in CODEBOOK:
        lanes = [((pat >> (2 * ln)) & 3) - 1 for ln in range(4)]
        assert sorted(map(abs, lanes)) == [0, 1, 1, 1] and max(lanes) <= 1
    assert len(set(CODEBOOK)) == 32
    for _ in range(10):
        t = np.zeros(256, np.int64)
        for grp in range(64):
            pat = CODEBOOK[RNG.integers(0, 32)]
            chunk, gloc = grp >> 4, grp & 15
            for ln in range(4):
                t[64 * chunk + gloc + 16 * ln] = ((pat >> (2 * ln)) & 3) - 1
        d = 2.0 ** RNG.integers(-8, 0)
        y = O.dequant(O.W_STQ1_0, enc_stq1_0(d, t), 1, 256)[0]
        assert np.array_equal(y, (t * d).astype(np.float32))


@pytest.mark.parametrize("wtype", [O.W_F32, O.W_F16, O.W_Q8_0, O.W_Q4_K, O.W_Q6_K, O.W_Q2_0C, O.W_STQ1_0])
def test_gemv_is_the_product_of_the_dequantized_rows(wtype):
    rows, cols = 5, 1024
    raw = RNG.integers(0, 256, O.row_bytes(wtype, cols) * rows, dtype=np.uint8)
    if wtype == O.W_F32:
        raw = RNG.standard_normal(rows * cols).astype(np.float32).view(np.uint8)
    elif wtype == O.W_F16:
        raw = RNG.standard_normal(rows * cols).astype(np.float16).view(np.uint8)
    x = RNG.standard_normal(cols).astype(np.float32)
    w = O.dequant(wtype, raw, rows, cols)
    ok = np.all(np.isfinite(w), axis=1)  # random fp16 scale bits may be inf/nan
    y = O.gemv(wtype, raw, rows, cols, x)
    ref = w.astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(y[ok], ref[ok], rtol=1e-6, atol=1e-6)
    y2 = O.gemv(wtype, raw, rows, cols, x, y=np.ones(rows, np.float32))
    assert np.allclose(y2[ok], ref[ok] + 1, rtol=1e-6, atol=1e-6)
