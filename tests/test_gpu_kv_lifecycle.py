"""GPU tests of the KV-cache lifecycle calls: the packed (parked) prefix has the engine's resize layout
(src/runtime/engine.cpp:248-275: per KV head the n positions in use, K values, V values, then K and V scales), a
pack / unpack round trip into a layer of another capacity restores the bytes exactly, and decode over the restored
layer is bit-identical to decode over the original."""
import numpy as np
import pytest
import torch

import qwengine_amd.ops as ops
from kvutil import KVTS, KV_NAMES, make_cache, seeded_normal

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
def test_pack_unpack_round_trip(gpu, kvt):
    n, cap, cap2 = 1000, 1200, 3000
    print(f"kv lifecycle kvt={KV_NAMES[kvt]} n={n}", flush=True)
    kv, _, _ = make_cache(kvt, n, cap, seed=71)
    nbytes = ops.kv_packed_bytes(kvt, n)
    dev = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    ops.kv_pack(kv, kvt, n, dev)
    ops.kv_pack(kv, kvt, n, host)
    torch.cuda.synchronize()
    # the layout: [K values][V values][K scales][V scales], each [4][n][row bytes]
    parts = [kv.k[:, :n], kv.v[:, :n]]
    if kv.ks is not None:
        parts += [kv.ks[:, :n].view(torch.uint8), kv.vs[:, :n].view(torch.uint8)]
    expect = torch.cat([p.contiguous().reshape(-1) for p in parts])
    assert expect.numel() == nbytes
    assert torch.equal(dev, expect)
    assert torch.equal(host, expect.cpu())

    kv2 = ops.KVLayer.allocate(kvt, cap2)
    ops.kv_unpack(host, kv2, kvt, n)
    torch.cuda.synchronize()
    assert torch.equal(kv2.k[:, :n], kv.k[:, :n]) and torch.equal(kv2.v[:, :n], kv.v[:, :n])
    if kv.ks is not None:
        assert torch.equal(kv2.ks[:, :n], kv.ks[:, :n]) and torch.equal(kv2.vs[:, :n], kv.vs[:, :n])

    q = seeded_normal((1, 24, 256), 72)
    gate = seeded_normal((1, 24, 256), 73)
    outs = []
    for layer in (kv, kv2):
        work = torch.empty(ops.attn_work_bytes(n) // 4 + 1, dtype=torch.float32, device="cuda")
        out = torch.empty((1, 24, 256), device="cuda")
        ops.attn_decode_multi(q, gate, layer, kvt, n - 1, 1, work, out)
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
