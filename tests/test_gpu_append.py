"""GPU parity of quantize-on-append, attention prep and the RoPE tables (bit-exact where the reference is exact).

Mirrors tests/kernels/test_ops.cu:278-287 (appended V rows == ggml quantizer values) and the quantizer edge cases of
tests/unit/test_quant_ref.cpp:119-122; prep against the double-precision restatement of test_ops.cu:260-272."""
import numpy as np
import pytest
import torch

import oracle as O
import qwengine_amd.ops as ops
from kvutil import KVTS, KV_NAMES, seeded_normal

pytestmark = pytest.mark.gpu


def _edge_rows(n, seed):
    """[n, 4, 256] rows: random at many scales plus the reference's edge cases."""
    rng = np.random.default_rng(seed)
    scales = 10.0 ** rng.uniform(-4, 4, size=(n, 4, 1))
    x = (rng.standard_normal((n, 4, 256)) * scales * (1 + np.arange(256) % 7)).astype(np.float32)
    x[0] = 0.0                                                    # all-zero rows
    x[1] = 0.0
    x[1, :, 3::32] = -5.0                                         # single -5 spike per block
    x[2] = np.float32(1e-30) * (np.arange(256) % 3)               # fp16 scale underflow
    x[3] = np.tile(np.array([3.0, -3.0] * 16, np.float32), 8)     # |x| ties: the first one sets the sign
    x[4] = np.tile(np.array([-3.0, 3.0] * 16, np.float32), 8)
    x[5] = (np.arange(256) % 32 - 16) * 0.5                       # exact halves (round-away vs round-even)
    x[6] = 127.0 * np.sign(np.sin(np.arange(256)))                # d = 1 exactly
    x[6, :, 1::32] = 2.5
    return x


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
def test_kv_append_bit_exact(gpu, oracle, kvt):
    n, cap, pos0 = 300, 512, 100
    xk = _edge_rows(n, 1)
    xv = _edge_rows(n, 2)[::-1].copy()
    kv = ops.KVLayer.allocate(kvt, cap)
    ops.kv_append(torch.from_numpy(xk).cuda(), torch.from_numpy(xv).cuda(), pos0, n, kvt, kv)
    torch.cuda.synchronize()
    for x, vals, sc in ((xk, kv.k, kv.ks), (xv, kv.v, kv.vs)):
        want_v, want_s = oracle.kv_store_rows(kvt, x.transpose(1, 0, 2).copy())  # [4, n, ...]
        got_v = vals[:, pos0:pos0 + n].cpu().numpy()
        assert np.array_equal(got_v, want_v), f"value bytes differ in {np.argwhere(got_v != want_v)[:5]}"
        if kvt != ops.F16:
            got_s = sc[:, pos0:pos0 + n].cpu().numpy().view(np.uint16)
            assert np.array_equal(got_s, want_s)
    # rows outside [pos0, pos0 + n) untouched
    assert not kv.k[:, :pos0].any() and not kv.v[:, pos0 + n:].any()


def _prep_inputs(n, seed):
    qg = seeded_normal((n, 24, 512), seed)
    k = seeded_normal((n, 4, 256), seed + 1)
    v = seeded_normal((n, 4, 256), seed + 2)
    g = torch.Generator(device="cuda").manual_seed(seed + 3)
    qn = 0.5 + torch.rand(256, generator=g, device="cuda")
    kn = 0.5 + torch.rand(256, generator=g, device="cuda")
    return qg, k, v, qn, kn


def _check_prep(oracle, kvt, kv, pos0, n, qg, k, v, qn, kn, q_out, gate, rope=None, rope_pos0=None, theta=1e7):
    eps = 1e-6
    if rope is None:
        qo, go, ko = oracle.attn_prep(qg.cpu().numpy(), k.cpu().numpy(), qn.cpu().numpy(), kn.cpu().numpy(),
                                      rope_pos0, theta, eps)
    else:
        qo, go, ko = oracle.attn_prep_table(qg.cpu().numpy(), k.cpu().numpy(), qn.cpu().numpy(), kn.cpu().numpy(),
                                            rope.cpu().numpy(), eps)
    assert np.array_equal(gate.cpu().numpy(), go)
    assert np.abs(q_out.cpu().numpy() - qo).max() <= 1e-5 * max(1.0, np.abs(qo).max())
    # V rows are stored unmodified: bytes equal the oracle quantizer of v (test_ops.cu:278-287)
    want_v, want_vs = oracle.kv_store_rows(kvt, v.cpu().numpy().transpose(1, 0, 2).copy())
    assert np.array_equal(kv.v[:, pos0:pos0 + n].cpu().numpy(), want_v)
    if kvt != ops.F16:
        assert np.array_equal(kv.vs[:, pos0:pos0 + n].cpu().numpy().view(np.uint16), want_vs)
    # K rows: the stored (normed, roped) row is the quantization of a value within float rounding of the oracle's
    kd = oracle.kv_load_rows(kvt, kv.k[:, pos0:pos0 + n].cpu().numpy(),
                             kv.ks[:, pos0:pos0 + n].cpu().numpy().view(np.uint16) if kv.ks is not None
                             else np.zeros((4, n, 8), np.uint16))
    kref = ko.transpose(1, 0, 2)
    if kvt == ops.F16:
        tol = np.abs(kref) * 2.0**-10 + 1e-6
    else:
        step = np.abs(kref).reshape(4, n, 8, 32).max(-1, keepdims=True) / (127.0 if kvt == ops.Q8_0 else 8.0)
        # half a step, plus the fp16 rounding of the scale times the largest code (Q8_0), or a full step where
        # Q4_0 clamps the top code
        frac = 0.6 if kvt == ops.Q8_0 else 1.05
        tol = np.broadcast_to(step * frac + 1e-5, (4, n, 8, 32)).reshape(4, n, 256)
    assert np.all(np.abs(kd - kref) <= tol)


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
def test_attn_prep_multi(gpu, oracle, kvt):
    n, pos0, rope_pos0, cap = 7, 1000, 262000, 1024
    qg, k, v, qn, kn = _prep_inputs(n, 40 + kvt)
    kv = ops.KVLayer.allocate(kvt, cap)
    q_out = torch.empty((n, 24, 256), device="cuda")
    gate = torch.empty_like(q_out)
    ops.attn_prep_multi(ops.RowSrc.device(qg, 12288), ops.RowSrc.device(k, 1024), ops.RowSrc.device(v, 1024), qn, kn,
                        pos0, rope_pos0, n, 1e7, 1e-6, kvt, kv, q_out, gate)
    torch.cuda.synchronize()
    _check_prep(oracle, kvt, kv, pos0, n, qg, k, v, qn, kn, q_out, gate, rope_pos0=rope_pos0)


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
def test_attn_prep_single(gpu, oracle, kvt):
    qg, k, v, qn, kn = _prep_inputs(1, 70 + kvt)
    kv = ops.KVLayer.allocate(kvt, 64)
    q_out = torch.empty((1, 24, 256), device="cuda")
    gate = torch.empty_like(q_out)
    ops.attn_prep(qg, k, v, qn, kn, 37, 1e7, 1e-6, kvt, kv, q_out, gate)
    torch.cuda.synchronize()
    _check_prep(oracle, kvt, kv, 37, 1, qg, k, v, qn, kn, q_out, gate, rope_pos0=37)


def test_rope_tables(gpu, oracle):
    B, p0, theta = 1000, 261000, 1e7
    rope = torch.empty((B, 64), device="cuda")
    ops.rope_table(p0, B, theta, rope)
    pos = np.stack([p0 + np.arange(B), p0 + np.arange(B) + 7, p0 + 3 * np.arange(B)], axis=1).astype(np.int32)
    rope_p = torch.empty((B, 64), device="cuda")
    ops.rope_table_pos(torch.from_numpy(pos).cuda(), B, theta, rope_p)
    torch.cuda.synchronize()
    assert np.abs(rope.cpu().numpy() - oracle.rope_table(p0, B, theta)).max() <= 1.2e-7
    assert np.abs(rope_p.cpu().numpy() - oracle.rope_table_pos(pos, theta)).max() <= 1.2e-7


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
def test_attn_prep_rows(gpu, oracle, kvt):
    B, p0, cap = 200, 500, 1024
    qg, k, v, qn, kn = _prep_inputs(B, 90 + kvt)
    rope = torch.empty((B, 64), device="cuda")
    ops.rope_table(p0, B, 1e7, rope)
    kv = ops.KVLayer.allocate(kvt, cap)
    q = torch.empty((B, 24, 256), device="cuda")
    gate = torch.empty_like(q)
    ops.attn_prep_rows(qg, k, v, qn, kn, B, p0, rope, 1e-6, kvt, kv, q, gate)
    torch.cuda.synchronize()
    _check_prep(oracle, kvt, kv, p0, B, qg, k, v, qn, kn, q, gate, rope=rope)


@pytest.mark.parametrize("kvt", [ops.Q8_0, ops.Q4_0], ids=lambda k: KV_NAMES[k])
def test_attn_prep_multi_host_tails(gpu, kvt):
    """RowSrc mapped-host tails (src/cuda/ops.cuh:24-34): row elements from `split` on come from pinned host rows of
    stride host_ld.  Q / gate split mid-head, K split mid-row, V entirely on the host: q, gate and the stored K / V
    bytes equal the all-device call's, and the device copies' NaN tails are never read."""
    n, pos0, rope_pos0 = 5, 300, 4000
    qg, k, v, qn, kn = _prep_inputs(n, 90 + kvt)

    def run(src_qg, src_k, src_v):
        kv = ops.KVLayer.allocate(kvt, 512)
        q_out = torch.empty((n, 24, 256), device="cuda")
        gate = torch.empty_like(q_out)
        ops.attn_prep_multi(src_qg, src_k, src_v, qn, kn, pos0, rope_pos0, n, 1e7, 1e-6, kvt, kv, q_out, gate)
        torch.cuda.synchronize()
        return kv, q_out, gate

    def split(t, width, at, pad):
        dev = t.clone().reshape(n, width)
        dev[:, at:] = float("nan")
        host = torch.full((n, width - at + pad), float("nan"), pin_memory=True)
        host[:, :width - at] = t.reshape(n, width)[:, at:].cpu()
        return ops.RowSrc(dev, at, host, width - at + pad), host

    kv0, q0, g0 = run(ops.RowSrc.device(qg, 12288), ops.RowSrc.device(k, 1024), ops.RowSrc.device(v, 1024))
    sq, hq = split(qg, 12288, 5000, 3)
    sk, hk = split(k, 1024, 300, 1)
    sv, hv = split(v, 1024, 0, 0)
    kv1, q1, g1 = run(sq, sk, sv)
    assert torch.equal(q0, q1) and torch.equal(g0, g1)
    assert torch.equal(kv0.k[:, pos0:pos0 + n], kv1.k[:, pos0:pos0 + n])
    assert torch.equal(kv0.v[:, pos0:pos0 + n], kv1.v[:, pos0:pos0 + n])
    assert torch.equal(kv0.ks[:, pos0:pos0 + n], kv1.ks[:, pos0:pos0 + n])
    assert torch.equal(kv0.vs[:, pos0:pos0 + n], kv1.vs[:, pos0:pos0 + n])
