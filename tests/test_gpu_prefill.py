"""GPU parity of causal prefill attention (fp16 MFMA kernel) against the float64 oracle on the stored cache, and
against the FP32 test kernel at the reference's chunk cases (tests/kernels/test_attn_prefill.cu:20-72: a cache of
1500 positions filled through rope_table + attn_prep_rows, chunks (p0, B) in {(0,37), (0,512), (300,129),
(1000,500), (1480,20)}), plus a 1300-token chunk (two passes of the kernel's 1024-token limit), chunks of 420 and 360
tokens (the kernel cuts their key ranges into 6 and 7 splits; 500 and 512 take 5, the rest 8), long-context chunks
of every format, the BASELINE 1024-token chunk at p0 = 32768 on all of its queries, and the ownership contract of
the workspace: the caller-owned form gives the drop-in call's bits, a captured HIP graph replays correctly, two
streams with their own workspaces do not interfere, a stream without a reservation gets one on first use (outside
graph capture), and a widened reservation keeps earlier captured graphs valid."""
import numpy as np
import pytest
import torch

import qwengine_amd.ops as ops
from kvutil import KVTS, KV_NAMES, assert_close, dequant_cache, make_cache, seeded_normal

pytestmark = pytest.mark.gpu

# (100, 900) and (480, 1000) run their pass as workgroups of 3 (row block, KV head, split) units, 900 tokens with a last
# workgroup of 2 units; (200, 1300) as a pass of 1024 such tokens and one of 276
CASES = [(0, 37), (0, 512), (300, 129), (1000, 500), (1480, 20), (200, 1300), (0, 420), (1100, 360), (100, 900),
         (480, 1000)]


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
    ~N(0,1); every query against the float64 oracle (OpenMP over (token, head))."""
    kvt, p0, B = ops.Q8_0, 32768, 1024
    kv, _, _ = make_cache(kvt, p0 + B, p0 + B, seed=44)
    q = seeded_normal((B, 24, 256), 45).half().float()
    gate = seeded_normal((B, 24, 256), 46)
    got = _prefill(ops.attn_prefill, kv, q, gate, B, p0)
    Kd, Vd = dequant_cache(kv, p0 + B)
    print("C4: oracle over all 1024 queries", flush=True)
    ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, p0, B)
    assert_close(got, ref, "C4 all queries")


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
def test_prefill_long_context(gpu, oracle, kvt):
    """A ragged chunk (300 tokens: the last row block is partial) at p0 = 40000 for every format: the image pass,
    the split ranges and the causal tail at long context, every query against the oracle.  Inputs as in config C4
    (Q fp16-representable, K / V ~N(0,1)): the kernel multiplies Q, K and P in fp16 like the reference's MMA kernel
    (src/cuda/prefill.cu:522-794); caches with outlier keys have their own test with the path's stated limit
    (test_prefill_outlier_keys_stated_limit)."""
    p0, B = 40000, 300
    print(f"prefill long context kvt={KV_NAMES[kvt]}", flush=True)
    kv, _, _ = make_cache(kvt, p0 + B, p0 + B + 16, seed=60 + 10 * kvt)  # K, V from seeds 60 + 10 kvt, + 1
    q = seeded_normal((B, 24, 256), 161).half().float()  # a seed of its own: q equal to cached keys is one-hot
    gate = seeded_normal((B, 24, 256), 162)
    got = _prefill(ops.attn_prefill, kv, q, gate, B, p0)
    Kd, Vd = dequant_cache(kv, p0 + B)
    ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, p0, B)
    assert_close(got, ref, f"prefill {KV_NAMES[kvt]} p0={p0} B={B}")


# Stated limit of the prefill path on caches with outlier keys.  The kernel multiplies fp16 K (d * code rounded to
# fp16 in the tile image), fp16 Q and fp16 P on the MFMA, as the reference's MMA kernel does
# (src/cuda/prefill.cu:522-794); on keys scaled x8 that rounding moves the output past the 2e-3 max-abs bar (the
# decode path takes exact K codes and a hi + lo Q instead).  Measured on this test's inputs: F16 max-abs 1.0e-3,
# rel-L2 2.1e-4 (F16 keys are exact in fp16: within the bar); Q8_0 6.6e-3 / 6.9e-4; Q4_0 5.1e-3 / 5.7e-4.  The rel-L2
# bar holds; max-abs is bounded here with margin:
PF_OUTLIER_MAX_ABS = 8e-3
PF_OUTLIER_REL_L2 = 1e-3


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
def test_prefill_outlier_keys_stated_limit(gpu, oracle, kvt):
    """A 300-token chunk at p0 = 40000 over a cache whose key rows are x8 at 1% of the (position, KV head) pairs (the
    C5 cache recipe), every query against the oracle: within the stated limit of the prefill path on such caches
    (PF_OUTLIER_MAX_ABS, PF_OUTLIER_REL_L2): the rel-L2 bar of outlier-free caches, a looser max-abs."""
    p0, B = 40000, 300
    print(f"prefill outlier keys kvt={KV_NAMES[kvt]}", flush=True)
    kv, _, _ = make_cache(kvt, p0 + B, p0 + B + 16, seed=260 + 10 * kvt, outlier_frac=0.01)
    q = seeded_normal((B, 24, 256), 361).half().float()
    gate = seeded_normal((B, 24, 256), 362)
    got = _prefill(ops.attn_prefill, kv, q, gate, B, p0)
    Kd, Vd = dequant_cache(kv, p0 + B)
    ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, p0, B)
    ma, rl = assert_close(got, ref, f"prefill outliers {KV_NAMES[kvt]}", PF_OUTLIER_MAX_ABS, PF_OUTLIER_REL_L2)
    print(f"prefill outlier keys kvt={KV_NAMES[kvt]}: max-abs {ma:.3e} rel-L2 {rl:.3e}", flush=True)


def _inputs(kvt, p0, B, seed):
    kv, _, _ = make_cache(kvt, p0 + B, p0 + B, seed=seed)
    q = seeded_normal((B, 24, 256), seed + 1)
    gate = seeded_normal((B, 24, 256), seed + 2)
    return kv, q, gate


def test_prefill_caller_workspace_matches(gpu):
    """attn_prefill_ws with a caller-owned workspace gives the drop-in call's bits; a short workspace is refused."""
    kvt, p0, B = ops.Q4_0, 3000, 200
    kv, q, gate = _inputs(kvt, p0, B, 70)
    want = _prefill(ops.attn_prefill, kv, q, gate, B, p0)
    nbytes = ops.attn_prefill_work_bytes(B, p0 + B)
    work = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    out = torch.empty((B, 24, 256), dtype=torch.float16, device="cuda")
    ops.attn_prefill_ws(q, gate, kv, kvt, B, p0, out, work)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), want.astype(np.float16).view(np.uint16))
    with pytest.raises(ops.QwaError, match="workspace"):
        ops.attn_prefill_ws(q, gate, kv, kvt, B, p0, out, work[:nbytes - 256])


def test_prefill_without_reservation_reserves_on_first_use(gpu):
    """The drop-in call needs no set-up call, as the reference's attn_prefill (src/cuda/prefill.cu:899-908): on a
    stream with no reservation, and past a reservation that is too small, it widens the stream's workspace itself and
    gives the caller-workspace bits."""
    kvt, p0, B = ops.Q8_0, 100, 16
    kv, q, gate = _inputs(kvt, p0, B, 80)
    work = torch.empty(ops.attn_prefill_work_bytes(B, p0 + B), dtype=torch.uint8, device="cuda")
    want = torch.empty((B, 24, 256), dtype=torch.float16, device="cuda")
    ops.attn_prefill_ws(q, gate, kv, kvt, B, p0, want, work)
    torch.cuda.synchronize()
    for reserve_first in (False, True):
        s = torch.cuda.Stream()
        out = torch.full((B, 24, 256), float("nan"), dtype=torch.float16, device="cuda")
        if reserve_first:
            ops.attn_prefill_reserve(B, 50, stream=s)  # too small a window: the call widens it
        torch.cuda.synchronize()
        ops.attn_prefill(q, gate, kv, kvt, B, p0, out, stream=s)
        s.synchronize()
        assert torch.equal(out, want), reserve_first
        ops.attn_prefill_release(stream=s)


def test_prefill_capture_beyond_reservation_is_refused(gpu):
    """Under graph capture a call the stream's workspace does not cover is refused (the graph would hold an
    allocation made inside the capture); the capture itself stays usable for other work."""
    kvt, p0, B = ops.Q8_0, 100, 16
    kv, q, gate = _inputs(kvt, p0, B, 82)
    s = torch.cuda.Stream()
    out = torch.empty((B, 24, 256), dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.graph(g, stream=s):
        try:
            ops.attn_prefill(q, gate, kv, kvt, B, p0, out, stream=s)
        except ops.QwaError as e:
            err = e
        out.zero_()
    assert err is not None and "capture" in str(err)
    g.replay()
    torch.cuda.synchronize()
    del g
    ops.attn_prefill_release(stream=s)


def test_prefill_growth_keeps_captured_graph_valid(gpu):
    """A graph captured with the stream's first workspace still replays correctly after a longer call has widened
    the reservation (the replaced workspace stays allocated until release)."""
    kvt, B = ops.Q8_0, 64
    kv, q, gate = _inputs(kvt, 4000, B, 84)
    want_short = _prefill(ops.attn_prefill, kv, q, gate, B, 200)
    want_long = _prefill(ops.attn_prefill, kv, q, gate, B, 4000)
    s = torch.cuda.Stream()
    ops.attn_prefill_reserve(B, 200 + B, stream=s)
    out = torch.full((B, 24, 256), float("nan"), dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        ops.attn_prefill(q, gate, kv, kvt, B, 200, out, stream=s)
    out2 = torch.empty_like(out)
    with torch.cuda.stream(s):
        ops.attn_prefill(q, gate, kv, kvt, B, 4000, out2, stream=s)  # widens the reservation
    s.synchronize()
    assert np.array_equal(out2.float().cpu().numpy(), want_long)
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.float().cpu().numpy(), want_short), f"replay {rep}"
    del g
    ops.attn_prefill_release(stream=s)


def test_prefill_reservations_widen(gpu):
    """Two reservations on one stream cover both maxima together: after (B 64, 300 positions) and (B 8, 2100
    positions) a call with B = 64 ending at 2100 runs in a workspace sized for both, with the caller-workspace bits."""
    kvt, p0, B = ops.Q8_0, 2036, 64
    kv, q, gate = _inputs(kvt, p0, B, 85)
    s = torch.cuda.Stream()
    out = torch.empty((B, 24, 256), dtype=torch.float16, device="cuda")
    ops.attn_prefill_reserve(64, 300, stream=s)
    ops.attn_prefill_reserve(8, 2100, stream=s)
    ops.attn_prefill(q, gate, kv, kvt, B, p0, out, stream=s)
    s.synchronize()
    work = torch.empty(ops.attn_prefill_work_bytes(B, p0 + B), dtype=torch.uint8, device="cuda")
    want = torch.empty_like(out)
    ops.attn_prefill_ws(q, gate, kv, kvt, B, p0, want, work)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    ops.attn_prefill_release(stream=s)


def test_prefill_in_hip_graph(gpu):
    """The drop-in call captured into a HIP graph on its first use (the workspace is reserved beforehand, nothing
    is allocated inside the call): every replay, with eager prefills of other inputs in between, equals the eager
    result bit for bit."""
    kvt, p0, B = ops.Q8_0, 2000, 160
    kv, q, gate = _inputs(kvt, p0, B, 90)
    kv2, q2, gate2 = _inputs(kvt, p0, B, 95)
    want = _prefill(ops.attn_prefill, kv, q, gate, B, p0)
    want2 = _prefill(ops.attn_prefill, kv2, q2, gate2, B, p0)
    s = torch.cuda.Stream()
    ops.attn_prefill_reserve(B, p0 + B, stream=s)
    out = torch.full((B, 24, 256), float("nan"), dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        ops.attn_prefill(q, gate, kv, kvt, B, p0, out, stream=s)
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.float().cpu().numpy(), want), f"replay {rep}"
        other = _prefill(ops.attn_prefill, kv2, q2, gate2, B, p0)  # eager work on the default stream in between
        assert np.array_equal(other, want2)
    del g
    ops.attn_prefill_release(stream=s)


def test_prefill_two_streams_do_not_interfere(gpu):
    """Two prefills queued concurrently on two streams, each with its own reserved workspace, give the bits of the
    same calls run one after the other."""
    kvt = ops.Q4_0
    cases = [(_inputs(kvt, 5000, 512, 100), 5000, 512), (_inputs(kvt, 7000, 384, 110), 7000, 384)]
    want = [_prefill(ops.attn_prefill, kv, q, g, B, p0) for (kv, q, g), p0, B in cases]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s, (_, p0, B) in zip(streams, cases):
        ops.attn_prefill_reserve(B, p0 + B, stream=s)
    outs = [torch.empty((B, 24, 256), dtype=torch.float16, device="cuda") for _, _, B in cases]
    torch.cuda.synchronize()
    for rep in range(4):
        for s, ((kv, q, g), p0, B), o in zip(streams, cases, outs):
            ops.attn_prefill(q, g, kv, kvt, B, p0, o, stream=s)
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert np.array_equal(o.float().cpu().numpy(), w), f"rep {rep}"
    for s in streams:
        ops.attn_prefill_release(stream=s)


def test_prefill_at_max_positions(gpu, oracle):
    """A 1024-token chunk ending at the largest supported position (262144), with a caller-owned workspace sized
    for it; a sample of 24 queries (every 43rd token plus the last) against the oracle."""
    kvt, n, B = ops.Q4_0, ops.attn_max_positions(), 1024
    p0 = n - B
    kv, _, _ = make_cache(kvt, n, n, seed=81)
    q = seeded_normal((B, 24, 256), 182).half().float()
    gate = seeded_normal((B, 24, 256), 183)
    work = torch.empty(ops.attn_prefill_work_bytes(B, n), dtype=torch.uint8, device="cuda")
    out = torch.empty((B, 24, 256), dtype=torch.float16, device="cuda")
    ops.attn_prefill_ws(q, gate, kv, kvt, B, p0, out, work)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    del work
    Kd, Vd = dequant_cache(kv, n)
    ts = list(range(0, B, 43)) + [B - 1]
    qn, gn = q.cpu().numpy(), gate.cpu().numpy()
    refs = np.stack([oracle.attention(qn[t:t + 1], gn[t:t + 1], Kd, Vd, p0 + t, 1)[0] for t in ts])
    assert_close(got[ts], refs, "prefill ending at 262144")


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
def test_prefill_random_sweep(gpu, oracle, kvt):
    """Seeded random chunks (p0, B) over one cache of 20000 positions, B in 1..1400 (one or two passes, 5 to 8 splits,
    units grouped per workgroup or not): every row against the FP32 test kernel (the reference's bound), the first and
    last 8 rows against the oracle."""
    n_pos = 20000
    rng = np.random.default_rng(4321 + kvt)
    kv, _, _ = make_cache(kvt, n_pos, n_pos, seed=80 + kvt)
    Kd, Vd = dequant_cache(kv, n_pos)
    for case in range(12):
        B = int(rng.integers(1, 1401))
        p0 = int(rng.integers(0, n_pos - B + 1))
        print(f"prefill random sweep kvt={KV_NAMES[kvt]} case={case} p0={p0} B={B}", flush=True)
        q = seeded_normal((B, 24, 256), 700 + 10 * case + kvt)
        gate = seeded_normal((B, 24, 256), 705 + 10 * case + kvt)
        got = _prefill(ops.attn_prefill, kv, q, gate, B, p0)
        simple = _prefill(ops.attn_prefill_simple, kv, q, gate, B, p0)
        assert np.abs(got - simple).max() / np.abs(simple).max() < 5e-3, (case, p0, B)
        for r0 in sorted({0, max(0, B - 8)}):
            nr = min(8, B - r0)
            ref = oracle.attention(q[r0:r0 + nr].cpu().numpy(), gate[r0:r0 + nr].cpu().numpy(), Kd, Vd, p0 + r0, nr)
            assert_close(got[r0:r0 + nr], ref, f"prefill random {KV_NAMES[kvt]} p0={p0} B={B} rows {r0}..")
