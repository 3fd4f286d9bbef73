"""Pins the CPU oracle (oracle/qwo.c) before it is trusted as the parity checker.

Every check here is independent of the oracle's own formulas: IEEE / numpy conversions, hand-computed known-answer
blocks (the edge cases of the reference's tests/unit/test_quant_ref.cpp:119-122), invariants that a dropped term,
wrong sign, wrong divisor or wrong rounding mode would break, and torch float64 attention as the library routine
the oracle must reduce to.
"""
import numpy as np
import pytest
import torch

import oracle as O


# ---------------------------------------------------------------------------------------------------- fp16
def test_fp16_exhaustive_round_trip(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = oracle.fp16_to_fp32(h)
    ok = ~np.isnan(f)
    back = oracle.fp32_to_fp16(f[ok])
    assert np.array_equal(back, h[ok])
    # and the values themselves are IEEE binary16 (numpy's conversion)
    assert np.array_equal(f[ok], h[ok].view(np.float16).astype(np.float32))


def test_fp32_to_fp16_matches_ieee_rne(oracle):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    # plus dense coverage of the fp16 subnormal / rounding boundaries
    edge = np.concatenate([
        np.float32(2.0) ** np.arange(-30, 17, dtype=np.float32),
        (np.arange(0, 4096, dtype=np.float32) + 0.5) * np.float32(2.0**-24),
        np.float32(65504.0) + np.arange(-32, 32, dtype=np.float32),
    ])
    x = np.concatenate([x, edge, -edge])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.fp32_to_fp16(x), want)


# ---------------------------------------------------------------------------------------------------- Q8_0
def _q8_block(blocks, b):
    d = blocks[34 * b:34 * b + 2].view(np.uint16)[0]
    qs = blocks[34 * b + 2:34 * b + 34].view(np.int8)
    return d, qs


def test_q8_0_known_answers(oracle):
    # all-zero block: d = 0, codes 0
    d, qs = _q8_block(oracle.quantize_q8_0(np.zeros(32, np.float32)), 0)
    assert d == 0 and not qs.any()
    # single -5 spike: d = fp16(5/127), code -127 there, 0 elsewhere
    x = np.zeros(32, np.float32)
    x[3] = -5.0
    d, qs = _q8_block(oracle.quantize_q8_0(x), 0)
    assert d == np.float16(np.float32(5.0) / np.float32(127.0)).view(np.uint16)
    assert qs[3] == -127 and np.count_nonzero(qs) == 1
    # amax 127 -> d = 1 exactly; halves round AWAY from zero (roundf), unlike round-half-even
    x = np.array([127, 2.5, -2.5, 0.5, -0.5, 1.5, 3.49, -126.5] + [0] * 24, np.float32)
    d, qs = _q8_block(oracle.quantize_q8_0(x), 0)
    assert d == 0x3C00
    assert list(qs[:8]) == [127, 3, -3, 1, -1, 2, 3, -127]
    # 1e-30 inputs: d underflows to an fp16 zero / subnormal, nothing blows up
    x = np.float32(1e-30) * (np.arange(32) % 3).astype(np.float32)
    d, qs = _q8_block(oracle.quantize_q8_0(x), 0)
    assert d == 0 and list(qs[:3]) == [0, 64, 127]


@pytest.mark.parametrize("scale", [1e-4, 1e-2, 1.0, 1e2, 1e4])
def test_q8_0_invariants(oracle, scale):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(32 * 500) * scale * (1 + np.arange(32 * 500) % 7)).astype(np.float32)
    blocks = oracle.quantize_q8_0(x)
    xb = x.reshape(-1, 32).astype(np.float64)
    d16 = blocks.reshape(-1, 34)[:, :2].copy().view(np.uint16)[:, 0]
    qs = blocks.reshape(-1, 34)[:, 2:].copy().view(np.int8).astype(np.int64)
    amax = np.abs(xb).max(axis=1)
    d32 = (amax.astype(np.float32) / np.float32(127)).astype(np.float64)
    assert np.array_equal(d16, (amax.astype(np.float32) / np.float32(127)).astype(np.float16).view(np.uint16))
    assert np.abs(qs).max() <= 127
    # the largest-magnitude element maps to +-127 with its sign
    i = np.abs(xb).argmax(axis=1)
    assert np.array_equal(qs[np.arange(len(i)), i], np.sign(xb[np.arange(len(i)), i]).astype(np.int64) * 127)
    # nearest integer of x / d (the fp32 reciprocal adds at most a few ulps)
    err = np.abs(xb / d32[:, None] - qs)
    assert err.max() <= 0.5 + 1e-4
    # monotone within a block
    for b in range(0, len(xb), 50):
        o = np.argsort(xb[b], kind="stable")
        assert np.all(np.diff(qs[b][o]) >= 0)
    # dequantized error: half a step plus the fp16 rounding of the scale (subnormal fp16 scales at small magnitudes)
    deq = oracle.dequantize_q8_0(blocks).reshape(-1, 32).astype(np.float64)
    d = d16.view(np.float16).astype(np.float64)
    bound = (0.5 + 1e-4) * d32[:, None] + np.abs(qs) * np.abs(d - d32)[:, None]
    assert np.all(np.abs(deq - xb) <= bound * (1 + 1e-6) + 1e-30)


# ---------------------------------------------------------------------------------------------------- Q4_0
def test_q4_0_known_answer_block(oracle):
    # x_j = ((5 j) % 16 - 8) / 2: first largest |x| is x_0 = -4 -> d = -4 / -8 = 0.5, code_j = (5 j) % 16
    j = np.arange(32)
    x = (((5 * j) % 16 - 8) * 0.5).astype(np.float32)
    blk = oracle.quantize_q4_0(x)
    assert blk[:2].view(np.uint16)[0] == 0x3800  # fp16(0.5)
    codes = (5 * j) % 16
    # ggml block order: element j in the low nibble, j + 16 in the high nibble of byte j
    assert list(blk[2:]) == [int(codes[i] | (codes[i + 16] << 4)) for i in range(16)]
    # split layout: element 2i low nibble, 2i + 1 high nibble of byte i
    x256 = np.tile(x, 8)
    vals, scales = oracle.kv_store_rows(O.Q4_0, x256[None])
    assert list(vals[0, :16]) == [int(codes[2 * i] | (codes[2 * i + 1] << 4)) for i in range(16)]
    assert np.all(scales[0] == 0x3800)


def test_q4_0_first_largest_sets_the_sign(oracle):
    x = np.zeros(32, np.float32)
    x[2], x[5] = 3.0, -3.0  # tie in |x|: the FIRST one (+3) is the max -> d = 3 / -8
    blk = oracle.quantize_q4_0(x)
    d = blk[:2].view(np.float16)[0]
    assert d == np.float16(-0.375)
    codes = np.array([(b & 15) for b in blk[2:]] + [(b >> 4) for b in blk[2:]])
    assert codes[2] == 0          # +3 / -0.375 + 8.5 = 0.5 -> 0
    assert codes[5] == 15         # -3 / -0.375 + 8.5 = 16.5 -> 16 -> clamped to 15
    assert codes[0] == 8          # 0 -> 8.5 -> 8


def test_q4_0_invariants(oracle):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(32 * 2000) * np.repeat(10.0 ** rng.uniform(-4, 4, 2000), 32)).astype(np.float32)
    blocks = oracle.quantize_q4_0(x).reshape(-1, 18)
    xb = x.reshape(-1, 32).astype(np.float64)
    d = blocks[:, :2].copy().view(np.float16)[:, 0].astype(np.float64)
    lo, hi = blocks[:, 2:] & 15, blocks[:, 2:] >> 4
    codes = np.concatenate([lo, hi], axis=1).astype(np.int64)
    assert codes.min() >= 0 and codes.max() <= 15
    first = np.abs(xb).argmax(axis=1)  # argmax returns the first maximum
    assert np.all(codes[np.arange(len(first)), first] == 0)
    assert np.all(np.sign(d) == -np.sign(xb[np.arange(len(first)), first]))
    deq = O.dequantize_q4_0(blocks.reshape(-1)).reshape(-1, 32).astype(np.float64)
    # away from the clamp, the code is the nearest level (fp16 scale and fp32 reciprocal give slack)
    inner = codes < 15
    err = np.abs(deq - xb)[inner] / np.abs(np.repeat(d[:, None], 32, 1))[inner]
    assert err.max() <= 0.5 + 5e-3


@pytest.mark.parametrize("kvt", [O.F16, O.Q8_0, O.Q4_0])
def test_split_layout_equals_ggml_blocks(oracle, kvt):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 256)).astype(np.float32) * 3
    x[0] = 0
    x[1, ::7] = -5
    vals, scales = oracle.kv_store_rows(kvt, x)
    got = oracle.kv_load_rows(kvt, vals, scales)
    if kvt == O.F16:
        want = x.astype(np.float16).astype(np.float32)
    elif kvt == O.Q8_0:
        want = oracle.dequantize_q8_0(oracle.quantize_q8_0(x)).reshape(x.shape)
    else:
        want = oracle.dequantize_q4_0(oracle.quantize_q4_0(x)).reshape(x.shape)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------------------------------------------- attention
def _torch_gated_attention(q, gate, K, V, pos0):
    """float64 SDPA with GQA expansion, causal offset pos0, scale 1/16, times sigmoid(gate)."""
    nq = q.shape[0]
    n = pos0 + nq
    qt = torch.from_numpy(q.astype(np.float64)).permute(1, 0, 2)          # [24, nq, 256]
    kt = torch.from_numpy(K[:, :n].astype(np.float64)).repeat_interleave(6, dim=0)  # [24, n, 256]
    vt = torch.from_numpy(V[:, :n].astype(np.float64)).repeat_interleave(6, dim=0)
    mask = torch.arange(n)[None, :] <= (pos0 + torch.arange(nq))[:, None]
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=1.0 / 16.0)
    o = o.permute(1, 0, 2).numpy()
    return o * (1.0 / (1.0 + np.exp(-gate.astype(np.float64))))


@pytest.mark.parametrize("pos0,nq", [(0, 1), (50, 5), (300, 7), (1000, 1)])
def test_attention_matches_torch_sdpa(oracle, pos0, nq):
    rng = np.random.default_rng(pos0 + nq)
    n = pos0 + nq
    q = rng.standard_normal((nq, 24, 256)).astype(np.float32)
    gate = rng.standard_normal((nq, 24, 256)).astype(np.float32)
    K = rng.standard_normal((4, n + 3, 256)).astype(np.float32)
    V = rng.standard_normal((4, n + 3, 256)).astype(np.float32)
    want = _torch_gated_attention(q, gate, K, V, pos0)
    got = oracle.attention(q, gate, K, V, pos0, nq, mode=0)
    assert np.abs(got - want).max() < 2e-6
    ref = oracle.attention(q, gate, K, V, pos0, nq, mode=1)  # the reference CPU arithmetic
    assert np.abs(ref - want).max() < 5e-5


def test_attention_closed_forms(oracle):
    rng = np.random.default_rng(1)
    n = 200
    q = rng.standard_normal((2, 24, 256)).astype(np.float32)
    gate = np.zeros((2, 24, 256), np.float32)
    K = rng.standard_normal((4, n, 256)).astype(np.float32)
    # constant V rows -> output = V * sigmoid(0) = V / 2
    V = np.broadcast_to(rng.standard_normal((4, 1, 256)).astype(np.float32), (4, n, 256)).copy()
    out = oracle.attention(q, gate, K, V, n - 2, 2)
    assert np.allclose(out, 0.5 * np.repeat(V[:, 0], 6, axis=0)[None], atol=1e-6)
    # q = 0 -> uniform weights -> mean of the visible V rows
    V = rng.standard_normal((4, n, 256)).astype(np.float32)
    out = oracle.attention(np.zeros_like(q), gate, K, V, 100, 2)
    for t in range(2):
        mean = V[:, :101 + t].astype(np.float64).mean(axis=1)
        assert np.allclose(out[t], 0.5 * np.repeat(mean, 6, axis=0), atol=1e-6)
    # needle: one key aligned with every query dominates; a stronger one past the causal window is invisible
    Kn = K * 0.01
    Kn[:, 70] = 50.0 * np.sign(q[0, ::6])
    Kn[:, 150] = 100.0 * np.sign(q[0, ::6])
    out = oracle.attention(q[:1], gate[:1], Kn, V, 120, 1)
    assert np.allclose(out[0, ::6], 0.5 * V[:, 70], atol=1e-5)  # the heads whose query the needle matches


# ---------------------------------------------------------------------------------------------------- prep / rope
def test_prep_matches_torch(oracle):
    rng = np.random.default_rng(9)
    n, pos0, theta, eps = 3, 123456, 1e7, 1e-6
    qg = rng.standard_normal((n, 24, 512)).astype(np.float32)
    k = rng.standard_normal((n, 4, 256)).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    q_out, gate, k_out = oracle.attn_prep(qg, k, qn, kn, pos0, theta, eps)
    assert np.array_equal(gate, qg[:, :, 256:])

    def ref(x, w, pos):
        x = torch.from_numpy(x.astype(np.float64))
        y = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * torch.from_numpy(w.astype(np.float64))
        inv = theta ** (-torch.arange(32, dtype=torch.float64) * 2 / 64)
        rot = torch.polar(torch.ones(32, dtype=torch.float64), pos * inv)
        z = torch.complex(y[..., :32], y[..., 32:64]) * rot
        y = y.clone()
        y[..., :32], y[..., 32:64] = z.real, z.imag
        return y.numpy()

    for r in range(n):
        assert np.allclose(q_out[r], ref(qg[r, :, :256], qn, pos0 + r), atol=2e-6, rtol=1e-6)
        assert np.allclose(k_out[r], ref(k[r], kn, pos0 + r), atol=2e-6, rtol=1e-6)
    # position 0: RoPE is the identity
    q0, _, _ = oracle.attn_prep(qg[:1], k[:1], qn, kn, 0, theta, eps)
    x = qg[0, :, :256].astype(np.float64)
    want = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * qn
    assert np.allclose(q0[0], want, atol=2e-6)


def test_rope_tables(oracle):
    p0, B, theta = 262000, 100, 1e7
    t = oracle.rope_table(p0, B, theta)
    i = np.arange(32)
    ang = np.mod((p0 + np.arange(B))[:, None] * theta ** (-2.0 * i / 64), 2 * np.pi)
    assert np.array_equal(t[:, :32], np.cos(ang).astype(np.float32)) or np.abs(t[:, :32] - np.cos(ang)).max() < 1e-7
    assert np.abs(t[:, 32:] - np.sin(ang)).max() < 1e-7
    pos = np.repeat((p0 + np.arange(B))[:, None], 3, axis=1)
    assert np.array_equal(oracle.rope_table_pos(pos, theta), t)  # text tokens: t = h = w
    pos[:, 1] += 5
    tp = oracle.rope_table_pos(pos, theta)
    assert np.array_equal(tp[:, 0], t[:, 0]) and not np.array_equal(tp[:, 1], t[:, 1])
    # the prep form with a table equals the form that computes its own angles
    rng = np.random.default_rng(2)
    qg = rng.standard_normal((B, 24, 512)).astype(np.float32)
    k = rng.standard_normal((B, 4, 256)).astype(np.float32)
    w = np.ones(256, np.float32)
    a = oracle.attn_prep_table(qg, k, w, w, t, 1e-6)
    b = oracle.attn_prep(qg, k, w, w, p0, theta, 1e-6)
    for x, y in zip(a, b):
        assert np.abs(x - y).max() < 1e-6


def test_act_q8_round_half_even(oracle):
    v = np.zeros(64, np.float32)
    v[:8] = [127, 2.5, -2.5, 3.5, 0.5, -1.5, 1.49, 0]
    v[32:] = np.linspace(-1, 1, 32, dtype=np.float32)
    q, d, s = oracle.act_q8(v)
    assert d[0] == 1.0
    assert list(q[:8]) == [127, 2, -2, 4, 0, -2, 1, 0]
    assert s[0] == np.float32(q[:32].astype(np.int64).sum())
    assert d[1] == np.float32(1.0) / np.float32(127.0)
    assert np.abs(q[32:] - v[32:] / d[1]).max() <= 0.5 + 1e-6
