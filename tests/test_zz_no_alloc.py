"""The allocation-free decode entry point (qwa_attn_decode_multi_noalloc, no reference counterpart) against
attn_decode_multi with a caller work buffer: bit-identical outputs and ActQ8 rows on two calls in a row, the second
with a smaller input (fewer positions and queries), so stale records of the first call must not leak into the
second."""
import pytest
import torch

import qwengine_amd.ops as ops
from kvutil import make_cache, seeded_normal

pytestmark = pytest.mark.gpu


def _pair(kv, kvt, pos0, nq, seed, with_q8):
    q = seeded_normal((nq, 24, 256), seed)
    gate = seeded_normal((nq, 24, 256), seed + 1)
    work = torch.empty(ops.attn_work_bytes(pos0 + nq) // 4 + 1, dtype=torch.float32, device="cuda")
    want = torch.empty((nq, 24, 256), device="cuda")
    got = torch.full((nq, 24, 256), float("nan"), device="cuda")
    oq_w = ops.ActQ8.allocate(nq * 6144) if with_q8 else None
    oq_g = ops.ActQ8.allocate(nq * 6144) if with_q8 else None
    ops.attn_decode_multi(q, gate, kv, kvt, pos0, nq, work, want, oq_w)
    ops.attn_decode_multi_noalloc(q, gate, kv, kvt, pos0, nq, got, oq_g)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (kvt, pos0, nq)
    if with_q8:
        assert torch.equal(oq_g.q, oq_w.q) and torch.equal(oq_g.d, oq_w.d) and torch.equal(oq_g.s, oq_w.s)


@pytest.mark.parametrize("kvt", [ops.Q4_0, ops.Q8_0, ops.F16], ids=["q4_0", "q8_0", "f16"])
def test_noalloc_decode_matches_work_buffer(gpu, kvt):
    print(f"noalloc decode kvt={kvt}", flush=True)
    kv, _, _ = make_cache(kvt, 20007, 20016, seed=300 + kvt)
    _pair(kv, kvt, 20000, 7, 310, True)   # first call: 20007 positions, 7 queries
    _pair(kv, kvt, 2999, 2, 320, False)   # second, smaller: 3001 positions, 2 queries


def test_noalloc_decode_rejects_what_the_scratch_cannot_hold(gpu):
    """The static scratch covers every call the decode accepts (a static_assert beside the array checks its size
    against the record layout), so the calls it cannot hold are exactly those the decode's own rules reject: more
    than 8 queries, contexts past 262144 positions."""
    kv, _, _ = make_cache(ops.Q4_0, 64, 64, seed=330)
    out = torch.empty((9, 24, 256), device="cuda")
    with pytest.raises(ops.QwaError, match="queries"):
        ops.attn_decode_multi_noalloc(out, out, kv, ops.Q4_0, 10, 9, out)
    with pytest.raises(ops.QwaError, match="262144"):
        ops.attn_decode_multi_noalloc(out, out, kv, ops.Q4_0, 262144, 1, out)
