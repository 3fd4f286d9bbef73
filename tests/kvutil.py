"""Shared helpers of the GPU parity tests: seeded synthetic caches and error metrics (test infrastructure)."""
import numpy as np
import torch

import oracle as O
import qwengine_amd.ops as ops

KVTS = [ops.F16, ops.Q8_0, ops.Q4_0]
KV_NAMES = {ops.F16: "f16", ops.Q8_0: "q8_0", ops.Q4_0: "q4_0"}

# parity bar of the path (floating point): max-abs and relative L2 against the FP32 / float64 oracle
MAX_ABS = 2e-3
REL_L2 = 1e-3


def seeded_normal(shape, seed, device="cuda"):
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32)


def make_cache(kvt, n_pos, capacity, seed, outlier_frac=0.0, device="cuda"):
    """K, V ~ N(0,1) rows [n_pos, 4, 256] appended through the GPU quantizer (bit-exact with the oracle's, see
    test_kv_append_bit_exact).  outlier_frac: that fraction of (position, kv head) key rows scaled by 8."""
    kv = ops.KVLayer.allocate(kvt, capacity, device=device)
    K = seeded_normal((n_pos, 4, 256), seed, device)
    V = seeded_normal((n_pos, 4, 256), seed + 1, device)
    if outlier_frac > 0:
        g = torch.Generator(device=device).manual_seed(seed + 2)
        mask = torch.rand((n_pos, 4), generator=g, device=device) < outlier_frac
        K[mask] *= 8.0
    ops.kv_append(K, V, 0, n_pos, kvt, kv)
    torch.cuda.synchronize()
    return kv, K, V


def dequant_cache(kv, n_pos):
    """The cache exactly as stored, dequantized on the host by the oracle: K, V float32 [4, n_pos, 256]."""
    out = []
    for vals, sc in ((kv.k, kv.ks), (kv.v, kv.vs)):
        v = vals[:, :n_pos].cpu().numpy()
        s = sc[:, :n_pos].cpu().numpy().view(np.uint16) if sc is not None else np.zeros((4, n_pos, 8), np.uint16)
        out.append(O.kv_load_rows(kv.kvt, v, s))
    return out


def errors(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = got - ref
    return float(np.abs(d).max()), float(np.linalg.norm(d) / max(np.linalg.norm(ref), 1e-30))


def assert_close(got, ref, what="", max_abs=MAX_ABS, rel_l2=REL_L2):
    ma, rl = errors(got, ref)
    assert ma <= max_abs and rl <= rel_l2, f"{what}: max-abs {ma:.3e} (tol {max_abs}), rel-L2 {rl:.3e} (tol {rel_l2})"
    return ma, rl


def c1_inputs(device="cuda"):
    """BASELINE config 1 (the CPU reference's decode case): F16 KV cache of 4096 positions, K / V ~N(0,1) post-RoPE
    cast to fp16 (round to nearest even, by the F16 append), q and gate logits ~N(0,1), one query at position 4095.
    The GPU parity test and bench.py's CPU baseline use these same tensors."""
    n = 4096
    kv = ops.KVLayer.allocate(ops.F16, n, device=device)
    K = seeded_normal((n, 4, 256), 501, device)
    V = seeded_normal((n, 4, 256), 502, device)
    ops.kv_append(K, V, 0, n, ops.F16, kv)
    q = seeded_normal((1, 24, 256), 503, device)
    gate = seeded_normal((1, 24, 256), 504, device)
    return kv, q, gate
