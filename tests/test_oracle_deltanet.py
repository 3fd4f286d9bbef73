"""Pins the CPU oracle's Gated DeltaNet core (oracle/qwo.c: qwo_deltanet, restating
src/reference/ref_model.cpp:169-256) before it is trusted as the parity checker of the HIP DeltaNet kernels.

The checks do not retype the oracle's loops: a float64 numpy restatement in matrix form (outer products, matrix-vector
products), the delta rule's defining property (with write strength 1 and no decay the updated state maps the key
exactly onto the value), the pure-decay limit, the conv window, chaining of calls, and the unit RMS of the gated norm.
"""
import numpy as np
import pytest

import oracle as O

CH, QK, VD, VH, KH, HD = O.DN_CH, O.DN_QK, O.DN_V, O.DN_VH, O.DN_KH, O.DN_HD
EPS = 1e-6


def layer(seed, T, S_scale=0.1):
    rng = np.random.default_rng(seed)
    return dict(
        qkv=rng.standard_normal((T, CH)).astype(np.float32),
        z=rng.standard_normal((T, VD)).astype(np.float32),
        b=rng.standard_normal((T, VH)).astype(np.float32),
        a=rng.standard_normal((T, VH)).astype(np.float32),
        conv_w=(0.5 * rng.standard_normal((CH, 4))).astype(np.float32),
        dt_bias=rng.standard_normal(VH).astype(np.float32),
        ssm_a=(-np.exp(0.5 * rng.standard_normal(VH))).astype(np.float32),
        ssm_norm=(1.0 + 0.1 * rng.standard_normal(HD)).astype(np.float32),
        conv_state=rng.standard_normal((3, CH)).astype(np.float32),
        S=(S_scale * rng.standard_normal((VH, HD, HD))).astype(np.float32),
    )


def run(L, **over):
    d = dict(L, **over)
    return O.deltanet(d["qkv"], d["z"], d["b"], d["a"], d["conv_w"], d["dt_bias"], d["ssm_a"], d["ssm_norm"], EPS,
                      d["conv_state"], d["S"])


def silu(x):
    return x / (1.0 + np.exp(-x))


def numpy_deltanet(L):
    """float64 matrix-form restatement: window as a (T + 3) x CH sequence, per head S^T k and k delta^T."""
    qkv = L["qkv"].astype(np.float64)
    T = qkv.shape[0]
    seq = np.concatenate([L["conv_state"].astype(np.float64), qkv], axis=0)  # [3 + T][CH]
    w = L["conv_w"].astype(np.float64)
    S = L["S"].astype(np.float64).copy()  # [h][i][j]
    o = np.zeros((T, VD))
    for t in range(T):
        conv = silu(np.einsum("kc,ck->c", seq[t:t + 4], w))
        q = conv[:QK].reshape(KH, HD)
        k = conv[QK:2 * QK].reshape(KH, HD)
        v = conv[2 * QK:].reshape(VH, HD)
        q = q / np.maximum(np.linalg.norm(q, axis=1, keepdims=True), EPS)
        k = k / np.maximum(np.linalg.norm(k, axis=1, keepdims=True), EPS)
        beta = 1.0 / (1.0 + np.exp(-L["b"][t].astype(np.float64)))
        x = L["a"][t].astype(np.float64) + L["dt_bias"]
        decay = np.exp(np.where(x > 20, x, np.log1p(np.exp(x))) * L["ssm_a"])
        for h in range(VH):
            kk, qq = k[h % KH], q[h % KH]
            Sd = decay[h] * S[h]
            S[h] = Sd + np.outer(kk, (v[h] - Sd.T @ kk) * beta[h])
            oh = (S[h].T @ qq) / np.sqrt(HD)
            oh = oh / np.sqrt(np.mean(oh * oh) + EPS) * L["ssm_norm"]
            o[t, h * HD:(h + 1) * HD] = oh * silu(L["z"][t, h * HD:(h + 1) * HD].astype(np.float64))
    return o, seq[-3:], S


def test_matches_float64_matrix_form(oracle):
    L = layer(1, 4)
    o, cs, S = run(L)
    o64, cs64, S64 = numpy_deltanet(L)
    assert np.array_equal(cs, cs64.astype(np.float32))
    assert np.abs(S - S64).max() < 1e-5 * max(1.0, np.abs(S64).max())
    assert np.abs(o - o64).max() < 2e-5 * max(1.0, np.abs(o64).max())


def test_delta_rule_writes_value_exactly(oracle):
    """beta = 1, decay = 1, identity-tap conv: afterwards S^T k_hat = v for every value head."""
    L = layer(2, 1)
    w = np.zeros((CH, 4), np.float32)
    w[:, 3] = 1.0  # conv output = silu(x)
    o, cs, S = run(L, conv_w=w, b=np.full((1, VH), 60.0, np.float32), ssm_a=np.zeros(VH, np.float32))
    conv = silu(L["qkv"][0].astype(np.float64))
    k = conv[QK:2 * QK].reshape(KH, HD)
    k = k / np.linalg.norm(k, axis=1, keepdims=True)
    v = conv[2 * QK:].reshape(VH, HD)
    for h in range(VH):
        got = S[h].astype(np.float64).T @ k[h % KH]
        assert np.abs(got - v[h]).max() < 1e-4 * max(1.0, np.abs(v[h]).max()), h


def test_zero_write_strength_only_decays(oracle):
    """beta -> 0 (sigmoid(-60) ~ 1e-26) and a + dt_bias = 0: S' = 2^A S (softplus(0) = ln 2)."""
    L = layer(3, 1)
    a = -L["dt_bias"][None, :].astype(np.float32)
    _, _, S = run(L, b=np.full((1, VH), -60.0, np.float32), a=a)
    want = (2.0 ** L["ssm_a"].astype(np.float64))[:, None, None] * L["S"].astype(np.float64)
    assert np.abs(S - want).max() < 1e-6


def test_conv_window_and_chaining(oracle):
    L = layer(4, 5)
    o, cs, S = run(L)
    assert np.array_equal(cs, L["qkv"][-3:])
    # the same tokens one call at a time, carrying conv window and state
    cs1, S1 = L["conv_state"], L["S"]
    outs = []
    for t in range(5):
        ot, cs1, S1 = run(L, qkv=L["qkv"][t:t + 1], z=L["z"][t:t + 1], b=L["b"][t:t + 1], a=L["a"][t:t + 1],
                          conv_state=cs1, S=S1)
        outs.append(ot)
    assert np.array_equal(np.concatenate(outs), o)
    assert np.array_equal(S1, S) and np.array_equal(cs1, cs)


def test_gated_norm_unit_rms(oracle):
    # no decay and state scale 3: the core output's mean square (~0.07) dwarfs eps, so before the weight and the
    # silu(z) gate every head row has RMS 1 - O(1e-5); z >= 0.5 keeps the gate away from zero in the ratio
    L = layer(5, 2, S_scale=3.0)
    o, _, _ = run(L, ssm_a=np.zeros(VH, np.float32), z=np.abs(L["z"]) + 0.5)
    g = silu((np.abs(L["z"]) + 0.5).astype(np.float64)).reshape(2, VH, HD) * L["ssm_norm"].astype(np.float64)
    r = o.reshape(2, VH, HD).astype(np.float64) / g
    rms = np.sqrt(np.mean(r * r, axis=2))
    assert np.abs(rms - 1.0).max() < 1e-3


def test_ba_row_stride(oracle):
    """b / a rows wider than 48 (the decode path's stride 64) read only the first 48 values."""
    L = layer(6, 2)
    o, _, S = run(L)
    pad = np.full((2, 16), 1e9, np.float32)
    o2, _, S2 = run(L, b=np.concatenate([L["b"], pad], 1), a=np.concatenate([L["a"], pad], 1))
    assert np.array_equal(o, o2) and np.array_equal(S, S2)
