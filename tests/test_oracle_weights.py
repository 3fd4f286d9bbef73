"""Pins the oracle's weight-format dequantizers (oracle/qwo.c: qwo_w_dequant_row, restating
src/quant/quant_ref.cpp:24-101,281-299) before they are trusted as the checker of the decode GEMV and the prefill
fp16 dequantizer.

Blocks are packed here from chosen scales, mins and codes by helpers that write ggml's byte layouts
(src/quant/quant_formats.h:92-104) directly; the dequantized values must then equal the format's formula evaluated on
those chosen fields, bit for bit.  A wrong byte offset, nibble, bit pair, scale index or sign fails.  Random blocks
are also checked against an independent vectorised numpy decoder, and the GEMV target against a float64 matmul.
"""
import numpy as np
import pytest

import oracle as O
from wutil import random_rows

F32 = np.float32


def h16(x):
    return np.float16(x).view(np.uint16)


def hval(bits):
    return np.uint16(bits).view(np.float16).astype(F32)


# ---- packers: fields -> ggml bytes ---------------------------------------------------------------------------------
def pack_q4k(d, dmin, s6, m6, codes):
    """d, dmin fp16 bits; s6, m6 [8] 6-bit; codes [256] 0..15"""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(dmin).tobytes(), np.uint8)
    sc = np.zeros(12, np.uint8)
    for j in range(4):
        sc[j] = (s6[j] & 63) | ((s6[j + 4] >> 4) << 6)
        sc[j + 4] = (m6[j] & 63) | ((m6[j + 4] >> 4) << 6)
        sc[j + 8] = (s6[j + 4] & 15) | ((m6[j + 4] & 15) << 4)
    b[4:16] = sc
    for j in range(8):
        for l in range(32):
            byte = 16 + 32 * (j // 2) + l
            b[byte] |= (codes[32 * j + l] & 15) << (4 * (j % 2))
    return b


def pack_q2k(d, dmin, s4, m4, codes):
    """s4, m4 [16] 4-bit; codes [256] 0..3: group g = weights 16 g .. 16 g + 15"""
    b = np.zeros(84, np.uint8)
    b[0:16] = (np.asarray(s4) & 15) | ((np.asarray(m4) & 15) << 4)
    for g in range(16):
        col, half, shift = g // 8, g % 2, 2 * ((g // 2) % 4)
        for l in range(16):
            b[16 + 32 * col + 16 * half + l] |= (codes[16 * g + l] & 3) << shift
    b[80:82] = np.frombuffer(np.uint16(d).tobytes(), np.uint8)
    b[82:84] = np.frombuffer(np.uint16(dmin).tobytes(), np.uint8)
    return b


def pack_q6k(d, sc8, codes):
    """sc8 [16] int8; codes [256] -32..31 (group of 16 = scale index)"""
    b = np.zeros(210, np.uint8)
    for k in range(256):
        c = int(codes[k]) + 32
        h, r, l = k // 128, (k % 128) // 32, k % 32
        lo = 64 * h + 32 * (r % 2) + l
        b[lo] |= (c & 15) << (4 if r >= 2 else 0)
        b[128 + 32 * h + l] |= (c >> 4) << (2 * r)
    b[192:208] = np.asarray(sc8, np.int8).view(np.uint8)
    b[208:210] = np.frombuffer(np.uint16(d).tobytes(), np.uint8)
    return b


def pack_iq4xs(d, ls, idx):
    """ls [8] 0..63 (scale = ls - 32); idx [256] 0..15 level indices"""
    b = np.zeros(136, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(d).tobytes(), np.uint8)
    sh = 0
    for j in range(8):
        sh |= ((ls[j] >> 4) & 3) << (2 * j)
        b[4 + j // 2] |= (ls[j] & 15) << (4 * (j % 2))
        for l in range(16):
            b[8 + 16 * j + l] = (idx[32 * j + l] & 15) | ((idx[32 * j + 16 + l] & 15) << 4)
    b[2:4] = np.frombuffer(np.uint16(sh).tobytes(), np.uint8)
    return b


IQ4_LEVELS = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int8)


# ---- known answers -------------------------------------------------------------------------------------------------
def test_q4k_known_answer(oracle):
    rng = np.random.default_rng(1)
    s6, m6 = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    codes = rng.integers(0, 16, 256)
    d, dmin = h16(0.0123), h16(0.0456)
    y = O.w_dequant(O.W_Q4_K, pack_q4k(d, dmin, s6, m6, codes), 256)[0]
    want = np.empty(256, F32)
    for k in range(256):
        j = k // 32
        want[k] = F32(hval(d) * F32(s6[j])) * F32(codes[k]) - F32(hval(dmin) * F32(m6[j]))
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_q2k_known_answer(oracle):
    rng = np.random.default_rng(2)
    s4, m4 = rng.integers(0, 16, 16), rng.integers(0, 16, 16)
    codes = rng.integers(0, 4, 256)
    d, dmin = h16(0.031), h16(-0.017)
    y = O.w_dequant(O.W_Q2_K, pack_q2k(d, dmin, s4, m4, codes), 256)[0]
    want = np.empty(256, F32)
    for k in range(256):
        g = k // 16
        want[k] = F32(hval(d) * F32(s4[g])) * F32(codes[k]) - F32(hval(dmin) * F32(m4[g]))
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_q6k_known_answer(oracle):
    rng = np.random.default_rng(3)
    sc8 = rng.integers(-128, 128, 16)
    codes = rng.integers(-32, 32, 256)
    d = h16(0.0077)
    y = O.w_dequant(O.W_Q6_K, pack_q6k(d, sc8, codes), 256)[0]
    want = np.array([F32(hval(d) * F32(sc8[k // 16])) * F32(codes[k]) for k in range(256)], F32)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_iq4xs_known_answer(oracle):
    rng = np.random.default_rng(4)
    ls = rng.integers(0, 64, 8)
    idx = rng.integers(0, 16, 256)
    d = h16(0.0021)
    y = O.w_dequant(O.W_IQ4_XS, pack_iq4xs(d, ls, idx), 256)[0]
    want = np.array([F32(hval(d) * F32(ls[k // 32] - 32)) * F32(IQ4_LEVELS[idx[k]]) for k in range(256)], F32)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_bf16_is_the_high_half(oracle):
    x = np.random.default_rng(5).standard_normal(64).astype(F32)
    bits = (x.view(np.uint32) >> 16).astype(np.uint16)
    y = O.w_dequant(O.W_BF16, bits.view(np.uint8), 64)[0]
    assert np.array_equal(y.view(np.uint32), bits.astype(np.uint32) << 16)


# ---- random blocks vs an independent vectorised decoder --------------------------------------------------------------
def np_dequant(fmt, W, K):
    """Vectorised numpy decoder written from the block layouts (one row)."""
    nb = K // 256
    if fmt == O.W_Q4_K:
        b = W.reshape(nb, 144)
        d, dmin = hval(b[:, 0:2].copy().view(np.uint16)[:, 0]), hval(b[:, 2:4].copy().view(np.uint16)[:, 0])
        sc = b[:, 4:16].astype(np.int32)
        s = np.concatenate([sc[:, 0:4] & 63, (sc[:, 8:12] & 15) | ((sc[:, 0:4] >> 6) << 4)], 1)
        m = np.concatenate([sc[:, 4:8] & 63, (sc[:, 8:12] >> 4) | ((sc[:, 4:8] >> 6) << 4)], 1)
        qs = b[:, 16:].reshape(nb, 4, 32).astype(np.int32)
        codes = np.stack([qs & 15, qs >> 4], 2).reshape(nb, 8, 32)
        dl = (d[:, None] * s.astype(F32)).astype(F32)
        ml = (dmin[:, None] * m.astype(F32)).astype(F32)
        return (dl[:, :, None] * codes.astype(F32) - ml[:, :, None]).astype(F32).reshape(-1)
    if fmt == O.W_Q2_K:
        b = W.reshape(nb, 84)
        sc = b[:, :16].astype(np.int32)
        qs = b[:, 16:80].reshape(nb, 2, 2, 16).astype(np.int32)  # [col][half][l]
        d, dmin = hval(b[:, 80:82].copy().view(np.uint16)[:, 0]), hval(b[:, 82:84].copy().view(np.uint16)[:, 0])
        shifts = np.array([0, 2, 4, 6])
        # codes[nb][col][shift][half][l] -> group g = 8 col + 2 j + half
        codes = (qs[:, :, None, :, :] >> shifts[None, None, :, None, None]) & 3
        codes = codes.reshape(nb, 16, 16)
        dl = (d[:, None] * (sc & 15).astype(F32)).astype(F32)
        ml = (dmin[:, None] * (sc >> 4).astype(F32)).astype(F32)
        return (dl[:, :, None] * codes.astype(F32) - ml[:, :, None]).astype(F32).reshape(-1)
    if fmt == O.W_Q6_K:
        b = W.reshape(nb, 210)
        ql = b[:, :128].reshape(nb, 2, 2, 32).astype(np.int32)  # [half][r & 1][l]
        qh = b[:, 128:192].reshape(nb, 2, 32).astype(np.int32)
        sc = b[:, 192:208].view(np.int8).astype(F32).reshape(nb, 2, 8)
        d = hval(b[:, 208:210].copy().view(np.uint16)[:, 0])
        out = np.empty((nb, 2, 4, 32), F32)
        for r in range(4):
            low = (ql[:, :, r % 2, :] >> (4 if r >= 2 else 0)) & 15
            high = (qh >> (2 * r)) & 3
            code = (low | (high << 4)) - 32
            scale = np.repeat(sc[:, :, 2 * r:2 * r + 2], 16, axis=2)
            out[:, :, r, :] = (d[:, None, None] * scale).astype(F32) * code.astype(F32)
        return out.reshape(-1)
    if fmt == O.W_IQ4_XS:
        b = W.reshape(nb, 136)
        d = hval(b[:, 0:2].copy().view(np.uint16)[:, 0])
        sh = b[:, 2:4].copy().view(np.uint16)[:, 0].astype(np.int32)
        sl = b[:, 4:8].astype(np.int32)
        j = np.arange(8)
        ls = ((sl[:, j // 2] >> (4 * (j % 2))) & 15) | (((sh[:, None] >> (2 * j)) & 3) << 4)
        qs = b[:, 8:].reshape(nb, 8, 16).astype(np.int32)
        lev = IQ4_LEVELS.astype(F32)[np.concatenate([qs & 15, qs >> 4], 2)]
        dl = (d[:, None] * (ls - 32).astype(F32)).astype(F32)
        return (dl[:, :, None] * lev).astype(F32).reshape(-1)
    raise ValueError(fmt)


@pytest.mark.parametrize("fmt", [O.W_Q2_K, O.W_Q4_K, O.W_Q6_K, O.W_IQ4_XS], ids=["q2_k", "q4_k", "q6_k", "iq4_xs"])
def test_random_blocks_match_vectorised_decoder(oracle, fmt):
    K = 1024
    W = random_rows(fmt, 4, K, 10 + fmt)
    got = O.w_dequant(fmt, W, K)
    for r in range(4):
        want = np_dequant(fmt, W[r], K)
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), (fmt, r)


@pytest.mark.parametrize("fmt", [O.W_Q4_K, O.W_IQ4_XS])
def test_gemv_ref_is_the_float64_product(oracle, fmt):
    K, N = 512, 37
    W = random_rows(fmt, N, K, 20 + fmt)
    x = np.random.default_rng(3).standard_normal((2, K)).astype(F32)
    q, d, _ = O.act_q8(x[0])
    q2, d2, _ = O.act_q8(x[1])
    q = np.stack([q, q2])
    d = np.stack([d, d2])
    y = O.gemv_ref(fmt, W, K, N, q, d)
    Wf = O.w_dequant(fmt, W, K).astype(np.float64)
    xhat = np.repeat(d.astype(np.float64), 32, axis=1) * q.astype(np.float64)
    assert np.allclose(y, xhat @ Wf.T, rtol=1e-12, atol=1e-12)


def test_unsupported_format_and_row_bytes(oracle):
    assert O.w_row_bytes(O.W_Q4_K, 5120) == 20 * 144
    assert O.w_row_bytes(O.W_Q6_K, 256) == 210
    assert O.w_row_bytes(O.W_Q4_K, 100) == 0
    assert O.w_row_bytes(29, 256) == 0  # IQ1_M: not restated


# ---- the i-quant grid formats (src/quant/quant_ref.cpp:105-222) ---------------------------------------------------
import hashlib  # noqa: E402
import json  # noqa: E402
import os  # noqa: E402

GRIDS = {}


def grid(name):
    """Expanded codebook as uint8 [entries][bytes] (pinned by test_iq_grids_match_reference_bytes)."""
    if name not in GRIDS:
        t, n, nb = O.IQ_TABLES[name]
        GRIDS[name] = np.frombuffer(O.iq_grid_bytes(name), np.uint8).reshape(n, nb)
    return GRIDS[name]


def test_iq_grids_match_reference_bytes(oracle):
    """The code words expand to the reference's byte tables (src/quant/iq_tables.inc:38-370): SHA-256 of each
    expanded table against tests/golden/iq_grids_sha256.json, written from the reference tables by
    tests/golden/make_iq_grids.py.  Plus the structure of the codebooks: entries distinct, bytes on the levels."""
    ref = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "iq_grids_sha256.json")))
    for name, want in ref.items():
        g = grid(name)
        assert g.shape == (want["entries"], want["bytes_per_entry"])
        assert hashlib.sha256(g.tobytes()).hexdigest() == want["sha256"], name
        assert len({bytes(r) for r in g}) == g.shape[0], name
    assert set(np.unique(grid("IQ2XXS"))) == {8, 25, 43}
    assert set(np.unique(grid("IQ3S"))) == set(range(1, 16, 2))
    assert np.array_equal(grid("IQ2XXS")[0], [8] * 8)  # the first entry of every IQ2 table is all-lowest


def ksigns(s7):
    """ggml's sign byte: 7 bits plus the parity bit that makes the count of negatives even."""
    s7 = int(s7) & 127
    return s7 | ((bin(s7).count("1") & 1) << 7)


def _put_u16(b, off, v):
    b[off:off + 2] = np.frombuffer(np.uint16(v).tobytes(), np.uint8)


def _put_u32(b, off, v):
    b[off:off + 4] = np.frombuffer(np.uint32(v).tobytes(), np.uint8)


def pack_iq2xxs(d, idx, s7, sc):
    """idx [8][4] 8-bit grid indices, s7 [8][4] 7-bit sign indices, sc [8] 4-bit scales"""
    b = np.zeros(66, np.uint8)
    _put_u16(b, 0, d)
    for ib in range(8):
        b[2 + 8 * ib:6 + 8 * ib] = idx[ib]
        _put_u32(b, 6 + 8 * ib, sum(int(s7[ib][l]) << (7 * l) for l in range(4)) | (int(sc[ib]) << 28))
    return b


def pack_iq2xs(d, idx, s7, sc):
    """idx [32] 9-bit, s7 [32], sc [8][2] 4-bit (first / second 16 weights of each 32)"""
    b = np.zeros(74, np.uint8)
    _put_u16(b, 0, d)
    for k in range(32):
        _put_u16(b, 2 + 2 * k, int(idx[k]) | (int(s7[k]) << 9))
    for ib in range(8):
        b[66 + ib] = int(sc[ib][0]) | (int(sc[ib][1]) << 4)
    return b


def pack_iq2s(d, idx, signs, sc):
    """idx [32] 10-bit, signs [32] sign bytes, sc [8][2]"""
    b = np.zeros(82, np.uint8)
    _put_u16(b, 0, d)
    for k in range(32):
        ib, l = divmod(k, 4)
        b[2 + k] = int(idx[k]) & 255
        b[34 + k] = signs[k]
        b[66 + ib] |= ((int(idx[k]) >> 8) & 3) << (2 * l)
    for ib in range(8):
        b[74 + ib] = int(sc[ib][0]) | (int(sc[ib][1]) << 4)
    return b


def pack_iq3xxs(d, idx, s7, sc):
    """idx [8][8] 8-bit (two per 8 weights), s7 [8][4], sc [8]"""
    b = np.zeros(98, np.uint8)
    _put_u16(b, 0, d)
    for ib in range(8):
        b[2 + 8 * ib:10 + 8 * ib] = idx[ib]
        _put_u32(b, 66 + 4 * ib, sum(int(s7[ib][l]) << (7 * l) for l in range(4)) | (int(sc[ib]) << 28))
    return b


def pack_iq3s(d, idx, signs, sc):
    """idx [8][8] 9-bit, signs [8][4] sign bytes, sc [8] 4-bit"""
    b = np.zeros(110, np.uint8)
    _put_u16(b, 0, d)
    for ib in range(8):
        for k in range(8):
            b[2 + 8 * ib + k] = int(idx[ib][k]) & 255
            b[66 + ib] |= ((int(idx[ib][k]) >> 8) & 1) << k
        b[74 + 4 * ib:78 + 4 * ib] = signs[ib]
        b[106 + ib // 2] |= int(sc[ib]) << (4 * (ib % 2))
    return b


def _expect(db_of, byte_of, sign_of):
    """weights k = 0..255: F32(db * byte) * (-1 if sign else 1), in the reference's float order"""
    out = np.empty(256, F32)
    for k in range(256):
        v = F32(F32(db_of(k)) * F32(byte_of(k)))
        out[k] = -v if sign_of(k) else v
    return out


def _check(fmt, blk, want):
    y = O.w_dequant(fmt, blk, 256)[0]
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), np.argwhere(y != want)[:5]


def test_iq2xxs_known_answer(oracle):
    rng = np.random.default_rng(31)
    idx, s7, sc = rng.integers(0, 256, (8, 4)), rng.integers(0, 128, (8, 4)), rng.integers(0, 16, 8)
    d = h16(0.0137)
    g = grid("IQ2XXS")
    db = lambda k: F32(F32(hval(d) * F32(0.5 + sc[k // 32])) * F32(0.25))
    _check(O.W_IQ2_XXS, pack_iq2xxs(d, idx, s7, sc),
           _expect(db, lambda k: g[idx[k // 32][(k % 32) // 8]][k % 8],
                   lambda k: (ksigns(s7[k // 32][(k % 32) // 8]) >> (k % 8)) & 1))


def test_iq2xs_known_answer(oracle):
    rng = np.random.default_rng(32)
    idx, s7, sc = rng.integers(0, 512, 32), rng.integers(0, 128, 32), rng.integers(0, 16, (8, 2))
    d = h16(-0.0211)
    g = grid("IQ2XS")
    db = lambda k: F32(F32(hval(d) * F32(0.5 + sc[k // 32][(k % 32) // 16])) * F32(0.25))
    _check(O.W_IQ2_XS, pack_iq2xs(d, idx, s7, sc),
           _expect(db, lambda k: g[idx[k // 8]][k % 8], lambda k: (ksigns(s7[k // 8]) >> (k % 8)) & 1))


def test_iq2s_known_answer(oracle):
    rng = np.random.default_rng(33)
    idx, signs, sc = rng.integers(0, 1024, 32), rng.integers(0, 256, 32), rng.integers(0, 16, (8, 2))
    d = h16(0.0093)
    g = grid("IQ2S")
    db = lambda k: F32(F32(hval(d) * F32(0.5 + sc[k // 32][(k % 32) // 16])) * F32(0.25))
    _check(O.W_IQ2_S, pack_iq2s(d, idx, signs, sc),
           _expect(db, lambda k: g[idx[k // 8]][k % 8], lambda k: (int(signs[k // 8]) >> (k % 8)) & 1))


def test_iq3xxs_known_answer(oracle):
    rng = np.random.default_rng(34)
    idx, s7, sc = rng.integers(0, 256, (8, 8)), rng.integers(0, 128, (8, 4)), rng.integers(0, 16, 8)
    d = h16(0.0071)
    g = grid("IQ3XXS")
    db = lambda k: F32(F32(hval(d) * F32(0.5 + sc[k // 32])) * F32(0.5))
    # weights 8 l + j: grid entry idx[2 l + j // 4], byte j % 4; sign bit j of the group's sign byte
    _check(O.W_IQ3_XXS, pack_iq3xxs(d, idx, s7, sc),
           _expect(db, lambda k: g[idx[k // 32][2 * ((k % 32) // 8) + (k % 8) // 4]][k % 4],
                   lambda k: (ksigns(s7[k // 32][(k % 32) // 8]) >> (k % 8)) & 1))


def test_iq3s_known_answer(oracle):
    rng = np.random.default_rng(35)
    idx, signs, sc = rng.integers(0, 512, (8, 8)), rng.integers(0, 256, (8, 4)), rng.integers(0, 16, 8)
    d = h16(0.0152)
    g = grid("IQ3S")
    db = lambda k: F32(hval(d) * F32(1 + 2 * sc[k // 32]))
    _check(O.W_IQ3_S, pack_iq3s(d, idx, signs, sc),
           _expect(db, lambda k: g[idx[k // 32][2 * ((k % 32) // 8) + (k % 8) // 4]][k % 4],
                   lambda k: (int(signs[k // 32][(k % 32) // 8]) >> (k % 8)) & 1))


def test_iq_sign_parity(oracle):
    """IQ2_XXS / IQ2_XS / IQ3_XXS: every group of 8 weights has an even number of negative values."""
    for fmt in (O.W_IQ2_XXS, O.W_IQ2_XS, O.W_IQ3_XXS):
        W = random_rows(fmt, 3, 1024, 40 + fmt)
        y = O.w_dequant(fmt, W, 1024).reshape(-1, 8)
        assert ((y < 0).sum(1) % 2 == 0).all(), fmt


def np_dequant_iq(fmt, W, K):
    """Vectorised numpy decoder of the grid formats, written from the block layouts (one row)."""
    nb = K // 256
    rb = O.w_row_bytes(fmt, 256)
    b = W.reshape(nb, rb)
    d = hval(b[:, 0:2].copy().view(np.uint16)[:, 0])
    par = np.array([ksigns(i) for i in range(128)], np.int64)
    bits8 = lambda s: ((s[..., None] >> np.arange(8)) & 1).astype(bool)
    if fmt in (O.W_IQ2_XXS, O.W_IQ3_XXS):
        if fmt == O.W_IQ2_XXS:
            q = b[:, 2:66].reshape(nb, 8, 8)
            idx, aux = q[:, :, :4].astype(np.int64), q[:, :, 4:8].copy().view(np.uint32)[..., 0].astype(np.int64)
            g = grid("IQ2XXS")[idx].reshape(nb, 8, 4, 8)
            db = (d[:, None] * (F32(0.5) + (aux >> 28).astype(F32))).astype(F32) * F32(0.25)
        else:
            idx = b[:, 2:66].reshape(nb, 8, 8).astype(np.int64)
            aux = b[:, 66:98].copy().view(np.uint32).reshape(nb, 8).astype(np.int64)
            g = grid("IQ3XXS")[idx].reshape(nb, 8, 4, 8)
            db = (d[:, None] * (F32(0.5) + (aux >> 28).astype(F32))).astype(F32) * F32(0.5)
        sg = bits8(par[(aux[..., None] >> (7 * np.arange(4))) & 127])          # [nb][8][4][8]
        dbw = np.broadcast_to(db.astype(F32)[:, :, None, None], sg.shape)
    elif fmt in (O.W_IQ2_XS, O.W_IQ2_S):
        if fmt == O.W_IQ2_XS:
            qs = b[:, 2:66].copy().view(np.uint16).reshape(nb, 8, 4).astype(np.int64)
            g = grid("IQ2XS")[qs & 511]
            sg = bits8(par[qs >> 9])
            sc = b[:, 66:74].astype(np.int64)
        else:
            qh = b[:, 66:74].astype(np.int64)
            idx = b[:, 2:34].reshape(nb, 8, 4).astype(np.int64) | (((qh[:, :, None] >> (2 * np.arange(4))) & 3) << 8)
            g = grid("IQ2S")[idx]
            sg = bits8(b[:, 34:66].reshape(nb, 8, 4).astype(np.int64))
            sc = b[:, 74:82].astype(np.int64)
        two = np.stack([sc & 15, sc >> 4], -1)                                   # [nb][8][2]
        db = ((d[:, None, None] * (F32(0.5) + two.astype(F32))).astype(F32) * F32(0.25)).astype(F32)
        dbw = np.broadcast_to(np.repeat(db, 2, axis=2)[:, :, :, None], sg.shape)
    else:  # IQ3_S
        qh = b[:, 66:74].astype(np.int64)
        idx = b[:, 2:66].reshape(nb, 8, 8).astype(np.int64) | (((qh[:, :, None] >> np.arange(8)) & 1) << 8)
        g = grid("IQ3S")[idx].reshape(nb, 8, 4, 8)
        sg = bits8(b[:, 74:106].reshape(nb, 8, 4).astype(np.int64))
        sc = b[:, 106:110].astype(np.int64)
        s4 = np.stack([sc & 15, sc >> 4], -1).reshape(nb, 8)
        db = (d[:, None] * (1 + 2 * s4).astype(F32)).astype(F32)
        dbw = np.broadcast_to(db[:, :, None, None], sg.shape)
    v = (dbw * g.astype(F32)).astype(F32)
    return np.where(sg, -v, v).astype(F32).reshape(-1)


IQ_FMTS = [O.W_IQ2_XXS, O.W_IQ2_XS, O.W_IQ2_S, O.W_IQ3_XXS, O.W_IQ3_S]


@pytest.mark.parametrize("fmt", IQ_FMTS, ids=["iq2_xxs", "iq2_xs", "iq2_s", "iq3_xxs", "iq3_s"])
def test_iq_random_blocks_match_vectorised_decoder(oracle, fmt):
    K = 1024
    W = random_rows(fmt, 4, K, 50 + fmt)
    got = O.w_dequant(fmt, W, K)
    for r in range(4):
        want = np_dequant_iq(fmt, W[r], K)
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), (fmt, r)


def test_iq_row_bytes(oracle):
    assert [O.w_row_bytes(f, 256) for f in IQ_FMTS] == [66, 74, 82, 98, 110]
    assert O.w_row_bytes(19, 256) == 0  # IQ1_S: not restated
