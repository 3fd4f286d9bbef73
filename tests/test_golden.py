"""The C oracle against the committed golden fixtures (tests/golden/make_golden.py: an independent numpy restatement
of the reference's quantizers, src/quant/quant_ref.cpp:507-538 in the split layout of src/cuda/common.cuh:54-80,
and of the float64 gated attention of src/reference/ref_model.cpp:138-163)."""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KVT = {"f16": 0, "q8_0": 1, "q4_0": 2}


def load(name):
    return np.load(os.path.join(GOLDEN, name))  # allow_pickle=False (default): plain arrays only


@pytest.mark.parametrize("name", ["f16", "q8_0", "q4_0"])
def test_oracle_quantizer_matches_golden(oracle, name):
    g = load("kv_quant_edge.npz")
    vals, scales = oracle.kv_store_rows(KVT[name], g["x"])
    assert np.array_equal(vals, g[f"{name}_vals"])
    if name != "f16":
        assert np.array_equal(scales, g[f"{name}_scales"])


@pytest.mark.parametrize("name", ["f16", "q8_0", "q4_0"])
def test_oracle_attention_matches_golden(oracle, name):
    g = load("attn_small.npz")
    kvt = KVT[name]
    K = g[f"{name}_K"].astype(np.float32).transpose(1, 0, 2).copy()  # [4, n, 256]
    V = g[f"{name}_V"].astype(np.float32).transpose(1, 0, 2).copy()
    Kd = oracle.kv_load_rows(kvt, *oracle.kv_store_rows(kvt, K))
    Vd = oracle.kv_load_rows(kvt, *oracle.kv_store_rows(kvt, V))
    pos0, nq = int(g[f"{name}_pos0"]), int(g[f"{name}_nq"])
    out = oracle.attention(g[f"{name}_q"].astype(np.float32), g[f"{name}_gate"].astype(np.float32), Kd, Vd, pos0, nq)
    np.testing.assert_allclose(out, g[f"{name}_out"], rtol=0, atol=1e-6)
    # the reference CPU arithmetic (fp32 dot products) stays well inside the path's tolerance
    out1 = oracle.attention(g[f"{name}_q"].astype(np.float32), g[f"{name}_gate"].astype(np.float32), Kd, Vd, pos0,
                            nq, mode=1)
    np.testing.assert_allclose(out1, g[f"{name}_out"], rtol=0, atol=1e-5)
