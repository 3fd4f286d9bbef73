"""GPU parity of decode / speculative-verify attention (split-K MFMA kernel + combine) against the float64 oracle
on the cache exactly as stored (the reference's own check, tests/kernels/test_ops.cu:288-337), the nq-independence
contract (memcmp, test_ops.cu:244-257), the FP32 test kernel, the ActQ8 epilogue, the long-context needle test
(test_ops.cu:354-423) and the BASELINE configurations at full size."""
import numpy as np
import pytest
import torch

import qwengine_amd.ops as ops
from kvutil import KVTS, KV_NAMES, assert_close, c1_inputs, dequant_cache, make_cache, seeded_normal

pytestmark = pytest.mark.gpu


def _qg(nq, seed):
    return seeded_normal((nq, 24, 256), seed), seeded_normal((nq, 24, 256), seed + 100)


def _decode(kv, q, gate, pos0, nq, oq=None):
    work = torch.empty(ops.attn_work_bytes(pos0 + nq) // 4 + 1, dtype=torch.float32, device="cuda")
    out = torch.empty((nq, 24, 256), device="cuda")
    ops.attn_decode_multi(q, gate, kv, kv.kvt, pos0, nq, work, out, oq)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
@pytest.mark.parametrize("n_pos", [1, 37, 300, 1000])
def test_decode_vs_oracle(gpu, oracle, kvt, n_pos):
    print(f"decode kvt={KV_NAMES[kvt]} n_pos={n_pos}", flush=True)
    kv, _, _ = make_cache(kvt, n_pos, 1024, seed=n_pos)
    q, gate = _qg(1, 5 + n_pos)
    out = _decode(kv, q, gate, n_pos - 1, 1)
    Kd, Vd = dequant_cache(kv, n_pos)
    ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, n_pos - 1, 1)
    assert_close(out.cpu().numpy(), ref, f"decode {KV_NAMES[kvt]} n_pos={n_pos}")
    # the FP32 test kernel (reference tolerance 5e-5 of max |ref|, test_ops.cu:339)
    out_s = torch.empty_like(out)
    ops.attn_decode_simple(q, gate, kv, kvt, n_pos, None, out_s)
    torch.cuda.synchronize()
    err = np.abs(out_s.cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= 5e-5, err


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
@pytest.mark.parametrize("n_pos", [8192, 8193, 8208, 8209])
def test_decode_class_chunk_counts(gpu, oracle, kvt, n_pos):
    """8192 positions are 512 chunks, one per residue class; 8193 and 8209 give class 0 (8209: also class 1) a second,
    one-key chunk, 8208 a full second chunk: a class's last chunk is not followed by a refill, whatever its count.
    Against the oracle, and one query of a 7-query call against the same query decoded alone, bit for bit."""
    print(f"decode class chunk counts kvt={KV_NAMES[kvt]} n_pos={n_pos}", flush=True)
    kv, _, _ = make_cache(kvt, n_pos, 16384, seed=n_pos)
    q, gate = _qg(7, 3 + n_pos)
    out = _decode(kv, q[:1].contiguous(), gate[:1].contiguous(), n_pos - 1, 1)
    Kd, Vd = dequant_cache(kv, n_pos)
    ref = oracle.attention(q[:1].cpu().numpy(), gate[:1].cpu().numpy(), Kd, Vd, n_pos - 1, 1)
    assert_close(out.cpu().numpy(), ref, f"decode {KV_NAMES[kvt]} n_pos={n_pos}")
    multi = _decode(kv, q, gate, n_pos - 7, 7).cpu().numpy()
    alone = _decode(kv, q[6:7].contiguous(), gate[6:7].contiguous(), n_pos - 1, 1).cpu().numpy()
    assert np.array_equal(multi[6:7].view(np.uint32), alone.view(np.uint32))


def test_config_c1_f16_4096(gpu, oracle):
    """single-token decode over an F16 cache of 4096 positions, on the tensors the CPU baseline
    times; against the float64 oracle and against the reference CPU arithmetic (oracle mode 1)."""
    kv, q, gate = c1_inputs()
    out = _decode(kv, q, gate, 4095, 1).cpu().numpy()
    Kd, Vd = dequant_cache(kv, 4096)
    qn, gn = q.cpu().numpy(), gate.cpu().numpy()
    assert_close(out, oracle.attention(qn, gn, Kd, Vd, 4095, 1), "C1 vs float64 oracle")
    assert_close(out, oracle.attention(qn, gn, Kd, Vd, 4095, 1, mode=1), "C1 vs reference CPU arithmetic")


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
@pytest.mark.parametrize("nq", [2, 3, 5, 7, 8])
def test_decode_multi_vs_oracle(gpu, oracle, kvt, nq):
    pos0 = 700
    print(f"verify kvt={KV_NAMES[kvt]} nq={nq}", flush=True)
    kv, _, _ = make_cache(kvt, pos0 + nq, 1024, seed=nq)
    q, gate = _qg(nq, 11 * nq)
    out = _decode(kv, q, gate, pos0, nq)
    Kd, Vd = dequant_cache(kv, pos0 + nq)
    ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, pos0, nq)
    assert_close(out.cpu().numpy(), ref, f"verify {KV_NAMES[kvt]} nq={nq}")


@pytest.mark.parametrize("kvt", [ops.Q4_0, ops.Q8_0], ids=lambda k: KV_NAMES[k])
@pytest.mark.parametrize("nq", [6, 7, 8])
def test_verify_chained_passes_bit_identical(gpu, oracle, kvt, nq):
    """Q4_0 / Q8_0 verify with 6..8 queries runs its two passes chained from 24576 / 12288 covered positions on (the
    one-tile pass's first chunks load while the two-tile pass merges, in two rounds) and unchained below.  Calls that
    end on either side of that boundary give every query the bits of the same query decoded alone, and the oracle's
    values."""
    print(f"verify chained passes kvt={KV_NAMES[kvt]} nq={nq}", flush=True)
    bound = 24576 if kvt == ops.Q4_0 else 12288
    n_pos = bound + 8
    kv, _, _ = make_cache(kvt, n_pos, 32768, seed=40 + nq)
    q, gate = _qg(8, 91 + nq)
    q, gate = q[:nq].contiguous(), gate[:nq].contiguous()
    Kd, Vd = dequant_cache(kv, n_pos)
    for end in (bound - 1, bound, bound + 8):  # positions the call covers: pos0 + nq
        pos0 = end - nq
        out = _decode(kv, q, gate, pos0, nq).cpu().numpy()
        ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, pos0, nq)
        assert_close(out, ref, f"verify {KV_NAMES[kvt]} nq={nq} end={end}")
        for t in range(nq):
            alone = _decode(kv, q[t:t + 1].contiguous(), gate[t:t + 1].contiguous(), pos0 + t, 1).cpu().numpy()
            assert np.array_equal(out[t].view(np.uint32), alone[0].view(np.uint32)), (end, t)


@pytest.mark.parametrize("kvt,nq", [(ops.F16, 7), (ops.F16, 6), (ops.Q8_0, 8)], ids=["f16-nq7", "f16-nq6", "q8_0-nq8"])
def test_verify_one_pass_boundary(gpu, oracle, kvt, nq):
    """F16 / Q8_0 verify with 6..8 queries takes the one-pass three-tile kernel (both half records of a record in one
    workgroup) from 12288 / 147456 covered positions on, the two passes in one launch below.  Calls that end on
    either side of that boundary give every query the bits of the same query decoded alone, and the oracle's
    values."""
    print(f"verify one-pass boundary kvt={KV_NAMES[kvt]} nq={nq}", flush=True)
    bound = 12288 if kvt == ops.F16 else 147456
    n_pos = bound + 8
    kv, _, _ = make_cache(kvt, n_pos, n_pos, seed=50 + nq)
    q, gate = _qg(nq, 97 + nq)
    Kd, Vd = dequant_cache(kv, n_pos)
    for end in (bound - 1, bound, bound + 8):  # positions the call covers: pos0 + nq
        pos0 = end - nq
        out = _decode(kv, q, gate, pos0, nq).cpu().numpy()
        ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, pos0, nq)
        assert_close(out, ref, f"verify {KV_NAMES[kvt]} nq={nq} end={end}")
        for t in range(nq):
            alone = _decode(kv, q[t:t + 1].contiguous(), gate[t:t + 1].contiguous(), pos0 + t, 1).cpu().numpy()
            assert np.array_equal(out[t].view(np.uint32), alone[0].view(np.uint32)), (end, t)


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
def test_decode_multi_is_bit_identical_to_single_calls(gpu, kvt):
    """decode_batch(n) == n x decode(), bit for bit (src/cuda/ops.cuh:134-135); split boundaries crossed on purpose."""
    base = 509  # queries straddle the 512-key split boundary
    kv, _, _ = make_cache(kvt, base + 8, 1024, seed=3)
    q, gate = _qg(8, 77)
    singles = [_decode(kv, q[t:t + 1].contiguous(), gate[t:t + 1].contiguous(), base + t, 1).cpu().numpy()
               for t in range(8)]
    for nq in range(1, 9):
        for t0 in (0, 8 - nq):
            out = _decode(kv, q[t0:t0 + nq].contiguous(), gate[t0:t0 + nq].contiguous(), base + t0, nq).cpu().numpy()
            for t in range(nq):
                assert np.array_equal(out[t].view(np.uint32), singles[t0 + t][0].view(np.uint32)), (nq, t0, t)


@pytest.mark.parametrize("kvt", [ops.Q8_0, ops.Q4_0], ids=lambda k: KV_NAMES[k])
def test_decode_actq8_epilogue(gpu, oracle, kvt):
    nq = 3
    kv, _, _ = make_cache(kvt, 400, 512, seed=9)
    q, gate = _qg(nq, 123)
    oq = ops.ActQ8.allocate(nq * 6144)
    out = _decode(kv, q, gate, 397, nq, oq)
    qw, dw, sw = oracle.act_q8(out.cpu().numpy())
    assert np.array_equal(oq.q.cpu().numpy(), qw)
    assert np.array_equal(oq.d.cpu().numpy(), dw)
    assert np.array_equal(oq.s.cpu().numpy(), sw)
    # the FP32 kernel's epilogue too
    oq1 = ops.ActQ8.allocate(6144)
    out1 = torch.empty((1, 24, 256), device="cuda")
    ops.attn_decode_simple(q[:1].contiguous(), gate[:1].contiguous(), kv, kvt, 398, None, out1, oq1)
    torch.cuda.synchronize()
    qw, dw, sw = oracle.act_q8(out1.cpu().numpy())
    assert np.array_equal(oq1.q.cpu().numpy(), qw) and np.array_equal(oq1.s.cpu().numpy(), sw)


def test_decode_long_context_needle(gpu, oracle):
    """140000-position Q8_0 cache with one key aligned with each group's first query at 135000
    (tests/kernels/test_ops.cu:354-423)."""
    n, needle, kvt = 140000, 135000, ops.Q8_0
    q, gate = _qg(1, 2024)
    K = seeded_normal((n, 4, 256), 31)
    V = seeded_normal((n, 4, 256), 32)
    K[needle] = 0.4 * q[0, ::6]
    kv = ops.KVLayer.allocate(kvt, n)
    ops.kv_append(K, V, 0, n, kvt, kv)
    out = _decode(kv, q, gate, n - 1, 1)
    Kd, Vd = dequant_cache(kv, n)
    ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, n - 1, 1)
    assert_close(out.cpu().numpy(), ref, "needle 140000")
    err = np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= 2e-3  # the reference's metric and tolerance


def test_config_c2_q8_decode_with_append(gpu, oracle):
    """Q8_0 cache of 4096 positions, the new token's K/V quantized on append, then decode."""
    kvt, n = ops.Q8_0, 4096
    kv, _, _ = make_cache(kvt, n, n + 1, seed=2)
    k_new = seeded_normal((1, 4, 256), 4242)
    v_new = seeded_normal((1, 4, 256), 4243)
    ops.kv_append(k_new, v_new, n, 1, kvt, kv)
    q, gate = _qg(1, 4244)
    out = _decode(kv, q, gate, n, 1)
    Kd, Vd = dequant_cache(kv, n + 1)
    # the appended rows are the oracle quantizer's, bit for bit
    import oracle as O
    want_v, _ = O.kv_store_rows(kvt, v_new.cpu().numpy()[0])
    assert np.array_equal(kv.v[:, n].cpu().numpy(), want_v)
    ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, n, 1)
    assert_close(out.cpu().numpy(), ref, "C2")


def test_config_c3_verify_q4_32768(gpu, oracle):
    """7 queries (causal within the block) over a Q4_0 cache of 32768 positions."""
    kvt, n, nq = ops.Q4_0, 32768, 7
    kv, _, _ = make_cache(kvt, n + nq, n + nq, seed=33)
    q, gate = _qg(nq, 3300)
    out = _decode(kv, q, gate, n, nq)
    Kd, Vd = dequant_cache(kv, n + nq)
    ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, n, nq)
    assert_close(out.cpu().numpy(), ref, "C3")


@pytest.mark.parametrize("nq", [1, 7])
def test_config_c5_long_decode_q4_150000(gpu, oracle, nq):
    """150000-position Q4_0 cache, 1% of key rows x8 (outliers), 1 query and 7-query verify."""
    kvt, n = ops.Q4_0, 150000
    kv, _, _ = make_cache(kvt, n, n, seed=55, outlier_frac=0.01)
    q, gate = _qg(nq, 5500 + nq)
    pos0 = n - nq
    out = _decode(kv, q, gate, pos0, nq)
    Kd, Vd = dequant_cache(kv, n)
    ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, pos0, nq)
    assert_close(out.cpu().numpy(), ref, f"C5 nq={nq}")


@pytest.mark.parametrize("kvt", [ops.Q4_0, ops.F16], ids=lambda k: KV_NAMES[k])
def test_decode_mapped_host_copy(gpu, kvt):
    """out_host (src/cuda/ops.cuh:136-137): the outputs are also written to mapped pinned host memory, fenced
    system-wide before the kernel ends, so they equal the device rows once the stream is synchronised; with the ActQ8
    epilogue at the same time."""
    nq, pos0 = 7, 2000
    kv, _, _ = make_cache(kvt, pos0 + nq, pos0 + nq, seed=41)
    q, gate = _qg(nq, 43)
    work = torch.empty(ops.attn_work_bytes(pos0 + nq) // 4 + 1, dtype=torch.float32, device="cuda")
    out = torch.empty((nq, 24, 256), device="cuda")
    host = torch.full((nq, 24, 256), float("nan"), pin_memory=True)
    oq = ops.ActQ8.allocate(nq * 6144)
    ops.attn_decode_multi(q, gate, kv, kvt, pos0, nq, work, out, oq, out_host=host)
    torch.cuda.synchronize()
    assert torch.equal(host, out.cpu())
    assert torch.equal(out, _decode(kv, q, gate, pos0, nq))


def test_decode_calls_on_two_streams(gpu):
    """Decode calls queued on two streams at once, each with its own work buffer, give the bits of the same calls
    made one after the other (the merge counters of concurrent calls are separate)."""
    kvt = ops.Q4_0
    cases = []
    for i, (n, nq) in enumerate(((30000, 1), (12000, 7))):
        kv, _, _ = make_cache(kvt, n + nq, n + nq, seed=51 + i)
        q, gate = _qg(nq, 53 + i)
        cases.append((kv, q, gate, n, nq))
    want = [_decode(kv, q, g, n, nq) for kv, q, g, n, nq in cases]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    works = [torch.empty(ops.attn_work_bytes(n + nq) // 4 + 1, dtype=torch.float32, device="cuda")
             for _, _, _, n, nq in cases]
    outs = [torch.empty_like(w) for w in want]
    torch.cuda.synchronize()
    for rep in range(5):
        for s, (kv, q, g, n, nq), w, o in zip(streams, cases, works, outs):
            ops.attn_decode_multi(q, g, kv, kvt, n, nq, w, o, stream=s)
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert torch.equal(o, w), rep


@pytest.mark.parametrize("kvt,n,nq", [(ops.Q4_0, 9000, 3), (ops.Q4_0, 9000, 7), (ops.F16, 33000, 7),
                                      (ops.Q4_0, 30000, 7), (ops.Q8_0, 20000, 8)],
                         ids=["q4_0-nq3", "q4_0-nq7-one-launch", "f16-nq7-three-tiles", "q4_0-nq7-chained",
                              "q8_0-nq8-chained"])
def test_decode_in_hip_graph(gpu, kvt, n, nq):
    """A decode step captured into a HIP graph (the engine's decode step): every replay, with eager decode calls in
    between, gives the eager bits; also the verify routes of 6..8 queries (two passes in one launch, unchained and
    chained, and the one-pass three-tile kernel with both half records in one workgroup)."""
    print(f"graph kvt={KV_NAMES[kvt]} n={n} nq={nq}", flush=True)
    kv, _, _ = make_cache(kvt, n + nq, n + nq, seed=61)
    q, gate = _qg(nq, 63)
    want = _decode(kv, q, gate, n, nq)
    work = torch.empty(ops.attn_work_bytes(n + nq) // 4 + 1, dtype=torch.float32, device="cuda")
    out = torch.empty_like(want)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        ops.attn_decode_multi(q, gate, kv, kvt, n, nq, work, out, stream=s)
    for rep in range(4):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
        assert torch.equal(_decode(kv, q, gate, n - 5, nq), _decode(kv, q, gate, n - 5, nq))
    del g


@pytest.mark.parametrize("kvt,nq,pos0", [(ops.F16, 7, 50000), (ops.F16, 4, 50000), (ops.Q8_0, 7, 50000),
                                         (ops.Q8_0, 5, 50000), (ops.Q8_0, 7, 220000), (ops.Q4_0, 7, 50000)],
                         ids=["f16-nq7", "f16-nq4", "q8_0-nq7", "q8_0-nq5", "q8_0-nq7-220k", "q4_0-nq7"])
def test_verify_passes_long_context(gpu, oracle, kvt, nq, pos0):
    """The verify kernels at a context with several chunks per class: F16 with 6..8 queries in its one-pass
    three-tile kernel (half records folded by the combine), 4..5 queries in the two-tile pass, Q8_0 7 queries as two
    passes in one launch at 50000 positions and in one pass at 220000, Q4_0 7 queries as two passes in one launch;
    against the oracle, and each query bit-identical to its one-query decode."""
    print(f"verify long context kvt={KV_NAMES[kvt]} nq={nq}", flush=True)
    kv, _, _ = make_cache(kvt, pos0 + nq, pos0 + nq, seed=90 + nq)
    q, gate = _qg(nq, 91 + nq)
    out = _decode(kv, q, gate, pos0, nq).cpu().numpy()
    Kd, Vd = dequant_cache(kv, pos0 + nq)
    ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, pos0, nq)
    assert_close(out, ref, f"verify {KV_NAMES[kvt]} nq={nq} at {pos0}")
    # a second context, with a partly filled last round of chunks
    if kvt == ops.F16 and nq >= 6:
        kv2, _, _ = make_cache(kvt, 30000 + nq, 30000 + nq, seed=93)
        q2, g2 = _qg(nq, 94)
        many = _decode(kv2, q2, g2, 30000, nq).cpu().numpy()
        one = _decode(kv2, q2[nq - 1:].contiguous(), g2[nq - 1:].contiguous(), 30000 + nq - 1, 1).cpu().numpy()
        assert np.array_equal(many[nq - 1].view(np.uint32), one[0].view(np.uint32))
    for t in range(nq):
        one = _decode(kv, q[t:t + 1].contiguous(), gate[t:t + 1].contiguous(), pos0 + t, 1).cpu().numpy()
        assert np.array_equal(out[t].view(np.uint32), one[0].view(np.uint32)), t


@pytest.mark.parametrize("kvt,nq", [(ops.Q4_0, 8), (ops.F16, 1), (ops.Q8_0, 3)],
                         ids=["q4_0-nq8", "f16-nq1", "q8_0-nq3"])
def test_decode_at_max_positions(gpu, oracle, kvt, nq):
    """The largest context the path supports (attn_max_positions = 262144; src/cuda/ops.cu:1002-1008): the last
    queries end exactly at position 262143, every record of the split is in use, against the oracle."""
    n = ops.attn_max_positions()
    print(f"decode at max positions kvt={KV_NAMES[kvt]} nq={nq}", flush=True)
    kv, _, _ = make_cache(kvt, n, n, seed=70 + kvt)
    q, gate = _qg(nq, 71 + nq)
    out = _decode(kv, q, gate, n - nq, nq)
    Kd, Vd = dequant_cache(kv, n)
    ref = oracle.attention(q.cpu().numpy(), gate.cpu().numpy(), Kd, Vd, n - nq, nq)
    assert_close(out.cpu().numpy(), ref, f"decode {KV_NAMES[kvt]} at {n} positions")
    with pytest.raises(ops.QwaError, match="262144"):
        _decode(kv, q, gate, n - nq + 1, nq)


def test_profile_window_stamps(gpu):
    """The opt-in timing window (qwa_profile_begin / end / device_ms / clock_mhz) over decode calls: one timed launch
    per call, event time >= device-clock time > 0, a shader clock in the range the MI355X runs at, and the calls' bits
    unchanged by the stamps."""
    kvt, n = ops.Q4_0, 20000
    kv, _, _ = make_cache(kvt, n + 1, n + 1, seed=91)
    q, gate = _qg(1, 93)
    want = _decode(kv, q, gate, n, 1)
    work = torch.empty(ops.attn_work_bytes(n + 1) // 4 + 1, dtype=torch.float32, device="cuda")
    out = torch.empty((1, 24, 256), device="cuda")
    ops.profile_begin()
    for _ in range(3):
        ops.attn_decode_multi(q, gate, kv, kvt, n, 1, work, out)
    ms, launches = ops.profile_end()
    dev_ms, mhz = ops.profile_device_ms(), ops.profile_clock_mhz()
    print(f"profile window: {launches} launches, {ms:.4f} ms events, {dev_ms:.4f} ms device, {mhz:.0f} MHz", flush=True)
    assert launches == 3
    assert ms >= dev_ms > 0.0
    assert 500.0 < mhz < 3500.0
    assert torch.equal(out, want)


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
def test_decode_verify_random_sweep(gpu, oracle, kvt):
    """Seeded random calls over one cache of 40968 positions, spanning every route below it (one-tile decode, two-tile
    pass, the two passes unchained and chained, the one-pass three-tile kernel for F16): nq in 1..8 and a random end.
    Each call gives every query the bits of the same query decoded alone (the nq-independence contract), and its last
    query the oracle's values."""
    n_pos = 40968
    rng = np.random.default_rng(1234 + kvt)
    kv, _, _ = make_cache(kvt, n_pos, n_pos, seed=60 + kvt)
    Kd, Vd = dequant_cache(kv, n_pos)
    for case in range(40):
        nq = int(rng.integers(1, 9))
        end = int(rng.integers(nq, n_pos + 1)) if case % 2 else int(rng.integers(nq, 4096))  # positions covered
        pos0 = end - nq
        print(f"random sweep kvt={KV_NAMES[kvt]} case={case} nq={nq} pos0={pos0}", flush=True)
        q, gate = _qg(nq, 500 + 10 * case + kvt)
        out = _decode(kv, q, gate, pos0, nq).cpu().numpy()
        for t in range(nq):
            alone = _decode(kv, q[t:t + 1].contiguous(), gate[t:t + 1].contiguous(), pos0 + t, 1).cpu().numpy()
            assert np.array_equal(out[t].view(np.uint32), alone[0].view(np.uint32)), (case, nq, pos0, t)
        ql, gl = q[nq - 1:].cpu().numpy(), gate[nq - 1:].cpu().numpy()
        ref = oracle.attention(ql, gl, Kd, Vd, pos0 + nq - 1, 1)
        assert_close(out[nq - 1:], ref, f"random sweep {KV_NAMES[kvt]} nq={nq} pos0={pos0}")
