"""Writes the committed golden fixtures of the hot path (test infrastructure; numpy only, run on the CPU).

The expected values here come from a second, independent restatement of the reference's semantics. It is written
directly in numpy float32 / float64 and shares no code with the C oracle. The fixtures therefore pin both the oracle
(tests/test_golden.py) and the HIP path (tests/test_gpu_golden.py) against a common set of vectors:

* kv_quant_edge.npz -- rows of 256 floats. They cover the reference quantizer test's edge cases
  (tests/unit/test_quant_ref.cpp:119-122: an all-zero row, a single -5 spike, 1e-30 magnitudes, scales 1e-4..1e4
  times (1 + i % 7)), plus |x| ties, exact halves and outliers. For each of F16 / Q8_0 / Q4_0 the fixture stores
  the split-layout bytes that kv_store_row must produce (src/cuda/common.cuh:54-80; the ggml rules of
  src/quant/quant_ref.cpp:507-538).
* attn_small.npz -- three small decode / verify cases (F16, Q8_0, Q4_0 with outlier keys). Each holds fp16-exact
  K/V/Q inputs, the gate logits, and the gated-attention output computed in float64 over the cache exactly as
  stored (src/reference/ref_model.cpp:138-163, src/cuda/ops.cu:507-815).

Usage: python tests/golden/make_golden.py   (rewrites both files; the output is deterministic)
"""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F16, Q8_0, Q4_0 = 0, 1, 2
VB = {F16: 512, Q8_0: 256, Q4_0: 128}


def _roundf(y: np.ndarray) -> np.ndarray:
    """C roundf (half away from zero) of float32 values, done in float64 so that |y| + 0.5 is exact."""
    a = np.floor(np.abs(y.astype(np.float64)) + 0.5)
    return np.copysign(a, y.astype(np.float64))


def store_row(kvt: int, x: np.ndarray):
    """One 256-float row -> (value bytes [VB], fp16 scale bits [8])."""
    x = np.asarray(x, np.float32)
    if kvt == F16:
        with np.errstate(over="ignore"):  # beyond 65504 -> inf, as the reference's round-to-nearest conversion
            return x.astype(np.float16).view(np.uint8).copy(), np.zeros(8, np.uint16)
    vals = np.zeros(VB[kvt], np.uint8)
    scales = np.zeros(8, np.uint16)
    for b in range(8):
        xb = x[32 * b:32 * b + 32]
        if kvt == Q8_0:
            amax = np.float32(np.max(np.abs(xb)))
            d = np.float32(amax / np.float32(127.0))
            inv = np.float32(1.0) / d if d != 0 else np.float32(0.0)
            q = _roundf(xb * inv).astype(np.int64)
            vals[32 * b:32 * b + 32] = (q & 0xFF).astype(np.uint8)
        else:
            # the signed value of the first element with the largest magnitude
            k = int(np.argmax(np.abs(xb)))  # argmax returns the first maximum
            mx = xb[k]
            d = np.float32(mx / np.float32(-8.0))
            inv = np.float32(1.0) / d if d != 0 else np.float32(0.0)
            t = (xb * inv).astype(np.float32) + np.float32(8.5)       # two roundings, no fused multiply-add
            q = np.minimum(15, np.trunc(t.astype(np.float64)).astype(np.int64))
            lo, hi = q[0::2], q[1::2]                                  # element 2i low nibble, 2i+1 high nibble
            vals[16 * b:16 * b + 16] = (lo | (hi << 4)).astype(np.uint8)
        scales[b] = np.float16(d).view(np.uint16)
    return vals, scales


def load_row(kvt: int, vals: np.ndarray, scales: np.ndarray) -> np.ndarray:
    if kvt == F16:
        return vals.view(np.float16).astype(np.float32)
    d = scales.view(np.float16).astype(np.float32)
    if kvt == Q8_0:
        q = vals.view(np.int8).astype(np.float32).reshape(8, 32)
    else:
        q = np.empty((8, 32), np.float32)
        v = vals.reshape(8, 16)
        q[:, 0::2] = (v & 0xF).astype(np.float32) - 8.0
        q[:, 1::2] = (v >> 4).astype(np.float32) - 8.0
    return (q * d[:, None]).astype(np.float32).reshape(256)


def edge_rows() -> np.ndarray:
    rng = np.random.default_rng(20240611)
    rows = []
    rows.append(np.zeros(256, np.float32))
    r = np.zeros(256, np.float32)
    r[3::32] = -5.0
    rows.append(r)
    rows.append((np.float32(1e-30) * (np.arange(256) % 3)).astype(np.float32))
    for e in range(-4, 5):
        rows.append((rng.standard_normal(256) * 10.0 ** e * (1 + np.arange(256) % 7)).astype(np.float32))
    rows.append(np.tile(np.array([3.0, -3.0] * 16, np.float32), 8))
    rows.append(np.tile(np.array([-3.0, 3.0] * 16, np.float32), 8))
    rows.append(((np.arange(256) % 32 - 16) * 0.5).astype(np.float32))
    r = (127.0 * np.sign(np.sin(np.arange(256)))).astype(np.float32)
    r[1::32] = 2.5
    rows.append(r)
    r = rng.standard_normal(256).astype(np.float32)
    r[17] = 40.0
    r[200] = -64.0
    rows.append(r)
    rows.append(np.full(256, 65504.0, np.float32))   # largest fp16: F16 exact, Q8_0 scale 515.78...
    rows.append(np.full(256, -1e-8, np.float32))     # fp16 subnormal scales
    return np.stack(rows)


def attention(q, gate, K, V, pos0, nq):
    """float64 gated GQA attention: q, gate [nq,24,256]; K, V [4, n, 256]; query t sees keys 0..pos0+t."""
    out = np.zeros((nq, 24, 256), np.float64)
    for t in range(nq):
        n = pos0 + t + 1
        for h in range(24):
            g = h // 6
            s = (K[g, :n].astype(np.float64) @ q[t, h].astype(np.float64)) / 16.0
            p = np.exp(s - s.max())
            o = (p @ V[g, :n].astype(np.float64)) / p.sum()
            out[t, h] = o / (1.0 + np.exp(-gate[t, h].astype(np.float64)))
    return out


def attn_case(kvt, n_pos, nq, seed, outlier_frac=0.0):
    rng = np.random.default_rng(seed)
    h16 = lambda a: a.astype(np.float16).astype(np.float32)   # fp16-exact inputs keep the fixture small
    K = h16(rng.standard_normal((n_pos, 4, 256)))
    V = h16(rng.standard_normal((n_pos, 4, 256)))
    if outlier_frac:
        K[rng.random((n_pos, 4)) < outlier_frac] *= 8.0
    q = h16(rng.standard_normal((nq, 24, 256)))
    gate = h16(rng.standard_normal((nq, 24, 256)))
    pos0 = n_pos - nq
    Kd = np.zeros((4, n_pos, 256), np.float32)
    Vd = np.zeros((4, n_pos, 256), np.float32)
    for g in range(4):
        for p in range(n_pos):
            Kd[g, p] = load_row(kvt, *store_row(kvt, K[p, g]))
            Vd[g, p] = load_row(kvt, *store_row(kvt, V[p, g]))
    out = attention(q, gate, Kd, Vd, pos0, nq)
    return dict(K=K.astype(np.float16), V=V.astype(np.float16), q=q.astype(np.float16), gate=gate.astype(np.float16),
                pos0=np.int32(pos0), nq=np.int32(nq), out=out.astype(np.float32))


def main():
    x = edge_rows()
    d = {"x": x}
    for kvt, name in ((F16, "f16"), (Q8_0, "q8_0"), (Q4_0, "q4_0")):
        vs = [store_row(kvt, r) for r in x]
        d[f"{name}_vals"] = np.stack([v for v, _ in vs])
        d[f"{name}_scales"] = np.stack([s for _, s in vs])
    np.savez_compressed(os.path.join(HERE, "kv_quant_edge.npz"), **d)

    a = {}
    for kvt, name, n_pos, nq, seed, of in ((F16, "f16", 9, 1, 11, 0.0), (Q8_0, "q8_0", 13, 2, 12, 0.0),
                                           (Q4_0, "q4_0", 29, 3, 13, 0.1)):
        for k, v in attn_case(kvt, n_pos, nq, seed, of).items():
            a[f"{name}_{k}"] = v
    np.savez_compressed(os.path.join(HERE, "attn_small.npz"), **a)


if __name__ == "__main__":
    main()
