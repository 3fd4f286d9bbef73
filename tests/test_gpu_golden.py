"""The HIP path against the committed golden fixtures (tests/golden/make_golden.py): quantize-on-append bytes
(bit-exact, src/cuda/common.cuh:54-80), and decode / verify / prefill outputs (max-abs 2e-3, rel-L2 1e-3) on the
fixture caches."""
import os

import numpy as np
import pytest
import torch

import qwengine_amd.ops as ops
from kvutil import assert_close

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KVT = {"f16": ops.F16, "q8_0": ops.Q8_0, "q4_0": ops.Q4_0}


@pytest.mark.parametrize("name", ["f16", "q8_0", "q4_0"])
def test_append_matches_golden_bytes(gpu, name):
    g = np.load(os.path.join(GOLDEN, "kv_quant_edge.npz"))
    x = g["x"]                                   # [R, 256]: use each row as K and V of all 4 KV heads
    R = x.shape[0]
    rows = torch.from_numpy(np.repeat(x[:, None, :], 4, axis=1).copy()).cuda()
    kv = ops.KVLayer.allocate(KVT[name], R + 3)
    ops.kv_append(rows, rows, 3, R, KVT[name], kv)
    torch.cuda.synchronize()
    for vals, sc in ((kv.k, kv.ks), (kv.v, kv.vs)):
        got = vals[:, 3:3 + R].cpu().numpy()
        for h in range(4):
            assert np.array_equal(got[h], g[f"{name}_vals"]), f"{name} head {h}"
            if name != "f16":
                assert np.array_equal(sc[h, 3:3 + R].cpu().numpy().view(np.uint16), g[f"{name}_scales"])


@pytest.mark.parametrize("name", ["f16", "q8_0", "q4_0"])
def test_attention_matches_golden(gpu, name):
    g = np.load(os.path.join(GOLDEN, "attn_small.npz"))
    kvt = KVT[name]
    K = torch.from_numpy(g[f"{name}_K"].astype(np.float32)).cuda()
    V = torch.from_numpy(g[f"{name}_V"].astype(np.float32)).cuda()
    n = K.shape[0]
    pos0, nq = int(g[f"{name}_pos0"]), int(g[f"{name}_nq"])
    q = torch.from_numpy(g[f"{name}_q"].astype(np.float32)).cuda()
    gate = torch.from_numpy(g[f"{name}_gate"].astype(np.float32)).cuda()
    want = g[f"{name}_out"]
    print(f"golden attention {name} n={n} nq={nq}", flush=True)
    kv = ops.KVLayer.allocate(kvt, 64)
    ops.kv_append(K, V, 0, n, kvt, kv)
    work = torch.empty(ops.attn_work_bytes(n) // 4 + 1, dtype=torch.float32, device="cuda")
    out = torch.empty((nq, 24, 256), device="cuda")
    ops.attn_decode_multi(q, gate, kv, kvt, pos0, nq, work, out)
    out16 = torch.empty((nq, 24, 256), dtype=torch.float16, device="cuda")
    ops.attn_prefill(q, gate, kv, kvt, nq, pos0, out16)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), want, f"decode {name}")
    assert_close(out16.float().cpu().numpy(), want, f"prefill {name}")
    # single-query calls give the same bits as the multi-query call
    for t in range(nq):
        o1 = torch.empty((1, 24, 256), device="cuda")
        ops.attn_decode_multi(q[t:t + 1], gate[t:t + 1], kv, kvt, pos0 + t, 1, work, o1)
        torch.cuda.synchronize()
        assert torch.equal(o1[0], out[t])
