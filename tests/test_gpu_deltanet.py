"""GPU parity of the Gated DeltaNet kernels (qwa_deltanet_step / _multi / _rows) against the CPU oracle
(oracle.deltanet, restating src/reference/ref_model.cpp:169-256).

Mirrors the reference's own check (tests/kernels/test_ops.cu:112-186: 6 decode steps from a zero state, outputs and
state within rel 2e-4, conv window exact) and adds: a non-zero starting state, the ActQ8 epilogue (bit-exact against
the oracle's quantization of the GPU output), the lazy-commit contract of deltanet_multi (a token sequence split into
calls with pending commits gives the same bits as one token per call, src/cuda/ops.cuh:93-95), write_after = 0,
mapped-host input tails and output copy, and the prefill rows path (fp16 output, state, conv window) including
core_out aliasing qkv.  The GPU state is [h][j][i] (j = value dim), the oracle's [h][i][j]."""
import numpy as np
import pytest
import torch

import qwengine_amd.ops as ops

pytestmark = pytest.mark.gpu

CH, VD, VH, HD = ops.DN_CH, ops.DN_VD, ops.DN_VH, ops.DN_HD
EPS = 1e-6
RTOL = 2e-4  # the reference's rel-err bound for outputs and state (test_ops.cu:177,183)


def rel_l2(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


class Layer:
    """Synthetic layer parameters (the reference test loads layer 0 of a model; none ships here) with both the
    oracle's and the GPU's copies of the conv window and state."""

    def __init__(self, seed, S_scale=0.0, cs_scale=0.0):
        rng = np.random.default_rng(seed)
        self.conv_w = (0.5 * rng.standard_normal((CH, 4))).astype(np.float32)
        self.dt_bias = rng.standard_normal(VH).astype(np.float32)
        self.ssm_a = (-np.exp(0.5 * rng.standard_normal(VH))).astype(np.float32)
        self.ssm_norm = (1.0 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
        self.cs = (cs_scale * rng.standard_normal((3, CH))).astype(np.float32)
        self.S = (S_scale * rng.standard_normal((VH, HD, HD))).astype(np.float32)  # [h][i][j]
        self.rng = rng

    def device(self, parity=0):
        cs2 = torch.zeros((2, 3, CH), dtype=torch.float32)
        cs2[parity] = torch.from_numpy(self.cs)
        S = torch.from_numpy(np.ascontiguousarray(self.S.transpose(0, 2, 1)))
        dev = lambda a: torch.as_tensor(a).contiguous().cuda()
        return ops.DNParams(dev(self.conv_w), dev(self.dt_bias), dev(self.ssm_a), dev(self.ssm_norm), cs2.cuda(),
                            S.cuda())

    def tokens(self, T):
        """Inputs shaped like the reference test's (qkv 0.5 N, z N, b N, a 2 N); b / a in rows of 64."""
        r = self.rng
        qkv = (0.5 * r.standard_normal((T, CH))).astype(np.float32)
        z = r.standard_normal((T, VD)).astype(np.float32)
        b = np.zeros((T, 64), np.float32)
        a = np.zeros((T, 64), np.float32)
        b[:, :VH] = r.standard_normal((T, VH))
        a[:, :VH] = 2.0 * r.standard_normal((T, VH))
        b[:, VH:] = np.nan  # the decode path reads only the first 48 of each row
        a[:, VH:] = np.nan
        return qkv, z, b, a

    def oracle(self, oracle, qkv, z, b, a, cs=None, S=None):
        return oracle.deltanet(qkv, z, b, a, self.conv_w, self.dt_bias, self.ssm_a, self.ssm_norm, EPS,
                               self.cs if cs is None else cs, self.S if S is None else S)


def gpu_state(p):
    return p.ssm_state.cpu().numpy().transpose(0, 2, 1)


def steps(p, qkv, z, b, a, parity0=0, oq=None):
    """One qwa_deltanet_step per token; returns the outputs [T][6144] and the parity after the last step."""
    outs = []
    par = parity0
    for t in range(qkv.shape[0]):
        o = torch.empty(VD, device="cuda")
        dq, dz = torch.from_numpy(qkv[t]).cuda(), torch.from_numpy(z[t]).cuda()
        db, da = torch.from_numpy(b[t, :VH].copy()).cuda(), torch.from_numpy(a[t, :VH].copy()).cuda()
        ops.deltanet_step(p, dq, dz, db, da, par, EPS, o, oq[t] if oq else None)
        torch.cuda.synchronize()
        outs.append(o.cpu().numpy())
        par ^= 1
    return np.stack(outs), par


@pytest.mark.parametrize("S_scale,cs_scale", [(0.0, 0.0), (0.1, 0.5)], ids=["zero_state", "random_state"])
def test_step_six_steps_vs_oracle(gpu, oracle, S_scale, cs_scale):
    print(f"deltanet_step S_scale={S_scale}", flush=True)
    L = Layer(11, S_scale, cs_scale)
    p = L.device(0)
    qkv, z, b, a = L.tokens(6)
    oq = [ops.ActQ8.allocate(VD) for _ in range(6)]
    out, par = steps(p, qkv, z, b, a, 0, oq)
    o_ref, cs_ref, S_ref = L.oracle(oracle, qkv, z, b[:, :VH], a[:, :VH])
    for t in range(6):
        assert rel_l2(out[t], o_ref[t]) < RTOL, t
        assert np.abs(out[t] - o_ref[t]).max() < 2e-3, t
        qw, dw, sw = oracle.act_q8(out[t])
        assert np.array_equal(oq[t].q.cpu().numpy(), qw), t
        assert np.array_equal(oq[t].d.cpu().numpy(), dw), t
        assert np.array_equal(oq[t].s.cpu().numpy(), sw), t
    assert rel_l2(gpu_state(p), S_ref) < RTOL
    assert par == 0  # six steps: the latest window is in buffer 0 again
    assert np.array_equal(p.conv_state[0].cpu().numpy(), cs_ref)
    # buffer 1 keeps the window written by the fifth step
    assert np.array_equal(p.conv_state[1].cpu().numpy(), np.concatenate([L.cs, qkv[:5]])[-3:])


def test_multi_lazy_commit_matches_steps_bitwise(gpu, oracle):
    """Speculative-decode pattern: call 1 emits 3 tokens and commits only the first (the rest saved to oqkv /
    obeta / oalpha); call 2 commits the 2 pending tokens and emits 3 new ones, committing all 5.  Every output,
    the state and the conv window equal one qwa_deltanet_step per token, bit for bit."""
    L = Layer(12, 0.1, 0.5)
    qkv, z, b, a = L.tokens(6)
    pa = L.device(0)
    out_a, par_a = steps(pa, qkv, z, b, a)

    pb = L.device(0)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    save_qkv = torch.full((3, CH), float("nan"), device="cuda")
    save_b = torch.full((3, 64), float("nan"), device="cuda")
    save_a = torch.full((3, 64), float("nan"), device="cuda")
    o1 = torch.empty((3, VD), device="cuda")
    oq1 = ops.ActQ8.allocate(3 * VD)
    t1 = ops.DNTokens(qkv=dev(qkv[:3]), z=dev(z[:3]), beta=dev(b[:3]), alpha=dev(a[:3]), oqkv=save_qkv, obeta=save_b,
                      oalpha=save_a)
    ops.deltanet_multi(pb, 0, t1, 0, 3, 1, EPS, o1, oq1)
    torch.cuda.synchronize()
    assert np.array_equal(save_qkv.cpu().numpy(), qkv[:3])
    assert np.array_equal(save_b.cpu().numpy()[:, :VH], b[:3, :VH])
    assert np.array_equal(save_a.cpu().numpy()[:, :VH], a[:3, :VH])
    o2 = torch.empty((3, VD), device="cuda")
    t2 = ops.DNTokens(sqkv=save_qkv[1:], sbeta=save_b[1:], salpha=save_a[1:], qkv=dev(qkv[3:]), z=dev(z[3:]),
                      beta=dev(b[3:]), alpha=dev(a[3:]))
    ops.deltanet_multi(pb, 1, t2, 2, 3, 5, EPS, o2)
    torch.cuda.synchronize()
    out_b = np.concatenate([o1.cpu().numpy(), o2.cpu().numpy()])
    assert np.array_equal(out_b.view(np.uint32), out_a.view(np.uint32))
    assert torch.equal(pb.ssm_state, pa.ssm_state)
    assert par_a == 0
    assert torch.equal(pb.conv_state[0], pa.conv_state[0])
    # the ActQ8 rows of call 1 (three tokens) equal the oracle's quantization of the same outputs
    qw, dw, sw = oracle.act_q8(o1.cpu().numpy())
    assert np.array_equal(oq1.q.cpu().numpy(), qw)
    assert np.array_equal(oq1.d.cpu().numpy(), dw) and np.array_equal(oq1.s.cpu().numpy(), sw)


def test_multi_write_after_zero_leaves_state(gpu):
    L = Layer(13, 0.1, 0.5)
    qkv, z, b, a = L.tokens(4)
    pa = L.device(0)
    out_a, _ = steps(pa, qkv, z, b, a)
    pb = L.device(0)
    S0, cs0 = pb.ssm_state.clone(), pb.conv_state.clone()
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    o = torch.empty((4, VD), device="cuda")
    ops.deltanet_multi(pb, 0, ops.DNTokens(qkv=dev(qkv), z=dev(z), beta=dev(b), alpha=dev(a)), 0, 4, 0, EPS, o)
    torch.cuda.synchronize()
    assert np.array_equal(o.cpu().numpy().view(np.uint32), out_a.view(np.uint32))
    assert torch.equal(pb.ssm_state, S0) and torch.equal(pb.conv_state, cs0)
    # n_commit + n_new = 0 does nothing
    ops.deltanet_multi(pb, 0, ops.DNTokens(), 0, 0, 0, EPS, None)
    torch.cuda.synchronize()
    assert torch.equal(pb.ssm_state, S0)


@pytest.mark.parametrize("qkv_split,z_split", [(5000, 3000), (0, 0), (2048, 6143)])
def test_multi_host_tails(gpu, qkv_split, z_split):
    """qkv channels >= qkv_split and z channels >= z_split read from pinned host rows (the device rows hold NaN
    there), outputs copied to a pinned host buffer: bit-identical to the all-device call."""
    print(f"deltanet_multi host split qkv={qkv_split} z={z_split}", flush=True)
    L = Layer(14, 0.1, 0.5)
    T = 5
    qkv, z, b, a = L.tokens(T)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    pa = L.device(1)
    oa = torch.empty((T, VD), device="cuda")
    ops.deltanet_multi(pa, 1, ops.DNTokens(qkv=dev(qkv), z=dev(z), beta=dev(b), alpha=dev(a)), 0, T, T, EPS, oa)

    pb = L.device(1)
    qd, zd = qkv.copy(), z.copy()
    qd[:, qkv_split:] = np.nan
    zd[:, z_split:] = np.nan
    qld, zld = CH - qkv_split + 3, VD - z_split + 1  # host row strides wider than the tails
    qh = torch.full((T, qld), float("nan"), pin_memory=True)
    zh = torch.full((T, zld), float("nan"), pin_memory=True)
    qh[:, :CH - qkv_split] = torch.from_numpy(qkv[:, qkv_split:])
    zh[:, :VD - z_split] = torch.from_numpy(z[:, z_split:])
    oh = torch.full((T, VD), float("nan"), pin_memory=True)
    ob = torch.empty((T, VD), device="cuda")
    tk = ops.DNTokens(qkv=dev(qd), z=dev(zd), beta=dev(b), alpha=dev(a), qkv_host=qh, qkv_split=qkv_split,
                      qkv_ld=qld, z_host=zh, z_split=z_split, z_ld=zld, o_host=oh)
    ops.deltanet_multi(pb, 1, tk, 0, T, T, EPS, ob)
    torch.cuda.synchronize()
    ref = oa.cpu().numpy().view(np.uint32)
    assert np.array_equal(ob.cpu().numpy().view(np.uint32), ref)
    assert np.array_equal(oh.numpy().view(np.uint32), ref)
    assert torch.equal(pb.ssm_state, pa.ssm_state)
    assert torch.equal(pb.conv_state[0], pa.conv_state[0])


def _rows(p, qkv, z, b, a, cin, alias=False):
    B = qkv.shape[0]
    dq = torch.from_numpy(np.ascontiguousarray(qkv)).cuda()
    dz = torch.from_numpy(np.ascontiguousarray(z)).cuda()
    db = torch.from_numpy(np.ascontiguousarray(b[:, :VH])).cuda()
    da = torch.from_numpy(np.ascontiguousarray(a[:, :VH])).cuda()
    work = torch.empty(ops.dn_work_bytes(B) // 4, dtype=torch.float32, device="cuda")
    core = dq if alias else torch.empty((B, VD), device="cuda")
    o16 = torch.empty((B, VD), dtype=torch.float16, device="cuda")
    ops.deltanet_rows(p, dq, dz, db, da, B, cin, EPS, work, core, o16)
    torch.cuda.synchronize()
    return o16.float().cpu().numpy()


@pytest.mark.parametrize("B,alias", [(1, False), (2, False), (17, True), (300, False)])
def test_rows_vs_oracle(gpu, oracle, B, alias):
    print(f"deltanet_rows B={B} alias={alias}", flush=True)
    L = Layer(20 + B, 0.1, 0.5)
    qkv, z, b, a = L.tokens(B)
    p = L.device(0)
    o = _rows(p, qkv, z, b, a, 0, alias)
    o_ref, cs_ref, S_ref = L.oracle(oracle, qkv, z, b[:, :VH], a[:, :VH])
    # fp16 output: within half an fp16 ulp of the rounded oracle plus the fp32 kernel's error
    assert rel_l2(o, o_ref) < 1e-3
    assert np.all(np.abs(o - o_ref) <= 2e-3 + 2.0 ** -11 * np.abs(o_ref))
    assert rel_l2(gpu_state(p), S_ref) < RTOL
    assert np.array_equal(p.conv_state[1].cpu().numpy(), cs_ref)
    assert np.array_equal(p.conv_state[0].cpu().numpy(), L.cs)  # the old window is left in place


def test_rows_then_decode_continues(gpu, oracle):
    """A 40-token prefill followed by 3 decode steps equals the oracle over all 43 tokens."""
    L = Layer(31, 0.0, 0.0)
    qkv, z, b, a = L.tokens(43)
    p = L.device(0)
    _rows(p, qkv[:40], z[:40], b[:40], a[:40], 0)
    out, _ = steps(p, qkv[40:], z[40:], b[40:], a[40:], parity0=1)
    o_ref, cs_ref, S_ref = L.oracle(oracle, qkv, z, b[:, :VH], a[:, :VH])
    for t in range(3):
        assert rel_l2(out[t], o_ref[40 + t]) < RTOL, t
    assert rel_l2(gpu_state(p), S_ref) < RTOL
    assert np.array_equal(p.conv_state[0].cpu().numpy(), cs_ref)


def test_multi_many_pending_matches_steps_bitwise(gpu):
    """6 pending + 7 new tokens in one call (more than one internal chunk of tokens) and a commit point inside the
    new tokens: outputs, state and conv window equal one step per token up to that point."""
    L = Layer(15, 0.1, 0.5)
    qkv, z, b, a = L.tokens(13)
    pa = L.device(0)
    steps(pa, qkv[:10], z[:10], b[:10], a[:10])  # the state and window after 10 tokens
    ref_after_all = L.device(0)
    out_all, _ = steps(ref_after_all, qkv, z, b, a)
    pb = L.device(0)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    o = torch.empty((7, VD), device="cuda")
    tk = ops.DNTokens(sqkv=dev(qkv[:6]), sbeta=dev(b[:6]), salpha=dev(a[:6]), qkv=dev(qkv[6:]), z=dev(z[6:]),
                      beta=dev(b[6:]), alpha=dev(a[6:]))
    ops.deltanet_multi(pb, 0, tk, 6, 7, 10, EPS, o)
    torch.cuda.synchronize()
    assert np.array_equal(o.cpu().numpy().view(np.uint32), out_all[6:].view(np.uint32))
    assert torch.equal(pb.ssm_state, pa.ssm_state)
    assert torch.equal(pb.conv_state[1], pa.conv_state[0])  # 10 steps from buffer 0 end in buffer 0
