"""GPU parity of causal prefill attention (fp16 MFMA kernel) against the float64 oracle on the stored cache, and
against the FP32 test kernel at the reference's chunk cases (tests/kernels/test_attn_prefill.cu:20-72: a cache of
1500 positions filled through rope_table + attn_prep_rows, chunks (p0, B) in {(0,37), (0,512), (300,129),
(1000,500), (1480,20)}), plus a 1300-token chunk (two passes of the kernel's 1024-token limit) and the BASELINE
1024-token chunk at p0 = 32768 on a sample of its queries."""
import numpy as np
import pytest
import torch

import qwengine_amd.ops as ops
from kvutil import KVTS, KV_NAMES, assert_close, dequant_cache, make_cache, seeded_normal

pytestmark = pytest.mark.gpu

CASES = [(0, 37), (0, 512), (300, 129), (1000, 500), (1480, 20), (200, 1300)]


@pytest.fixture(scope="module", params=KVTS, ids=lambda k: KV_NAMES[k])
def filled(request, gpu):
    """1500 positions through the real prep path (rope_table + attn_prep_rows), norm weights = 1."""
    kvt = request.param
    tot, cap = 1500, 2048
    qg = seeded_normal((tot, 24, 512), 11)
    k = seeded_normal((tot, 4, 256), 12)
    v = seeded_normal((tot, 4, 256), 13)
    w = torch.ones(256, device="cuda")
    rope = torch.empty((tot, 64), device="cuda")
    ops.rope_table(0, tot, 1e7, rope)
    kv = ops.KVLayer.allocate(kvt, cap)
    q = torch.empty((tot, 24, 256), device="cuda")
    gate = torch.empty_like(q)
    ops.attn_prep_rows(qg, k, v, w, w, tot, 0, rope, 1e-6, kvt, kv, q, gate)
    torch.cuda.synchronize()
    Kd, Vd = dequant_cache(kv, tot)
    return kvt, kv, q, gate, Kd, Vd


def _prefill(fn, kv, q, gate, B, p0):
    out = torch.empty((B, 24, 256), dtype=torch.float16, device="cuda")
    fn(q, gate, kv, kv.kvt, B, p0, out)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("p0,B", CASES)
def test_prefill_chunks(filled, oracle, p0, B):
    kvt, kv, q, gate, Kd, Vd = filled
    print(f"prefill kvt={KV_NAMES[kvt]} p0={p0} B={B}", flush=True)
    qc = q[p0:p0 + B].contiguous()
    gc = gate[p0:p0 + B].contiguous()
    got = _prefill(ops.attn_prefill, kv, qc, gc, B, p0)
    ref = oracle.attention(qc.cpu().numpy(), gc.cpu().numpy(), Kd, Vd, p0, B)
    assert_close(got, ref, f"prefill {KV_NAMES[kvt]} p0={p0} B={B}")
    simple = _prefill(ops.attn_prefill_simple, kv, qc, gc, B, p0)
    # the reference's comparison: tensor-core path vs the FP32 kernel, max diff / max |.| < 5e-3
    assert np.abs(got - simple).max() / np.abs(simple).max() < 5e-3
    assert_close(simple, ref, "prefill_simple", max_abs=1e-3, rel_l2=6e-4)  # fp16 output rounding only


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
def test_prefill_is_decode_consistent(gpu, oracle, kvt):
    """A prefill chunk's last query equals the decode of that query (both within tolerance of the same oracle)."""
    p0, B = 200, 64
    kv, _, _ = make_cache(kvt, p0 + B, 512, seed=21)
    q = seeded_normal((B, 24, 256), 22)
    gate = seeded_normal((B, 24, 256), 23)
    got = _prefill(ops.attn_prefill, kv, q, gate, B, p0)
    Kd, Vd = dequant_cache(kv, p0 + B)
    ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, p0, B)
    assert_close(got, ref, "prefill")


def test_config_c4_prefill_1024_at_32768(gpu, oracle):
    """1024 new tokens at p0 = 32768 over a Q8_0 cache (33792 positions), Q fp16-representable
    ~N(0,1); checked on 40 sampled queries (every KV head / tile position) against the float64 oracle."""
    kvt, p0, B = ops.Q8_0, 32768, 1024
    kv, _, _ = make_cache(kvt, p0 + B, p0 + B, seed=44)
    q = seeded_normal((B, 24, 256), 45).half().float()
    gate = seeded_normal((B, 24, 256), 46)
    got = _prefill(ops.attn_prefill, kv, q, gate, B, p0)
    Kd, Vd = dequant_cache(kv, p0 + B)
    rng = np.random.default_rng(4)
    ts = sorted(set([0, 1, 15, 16, 127, 128, 511, 1023] + list(rng.choice(B, 32, replace=False))))
    qn, gn = q.cpu().numpy(), gate.cpu().numpy()
    refs = np.stack([oracle.attention(qn[t:t + 1], gn[t:t + 1], Kd, Vd, p0 + t, 1)[0] for t in ts])
    assert_close(got[ts], refs, "C4 sampled queries")
