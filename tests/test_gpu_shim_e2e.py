"""The drop-in C++ boundary on the GPU: tests/shim_e2e.cpp calls the reference's operator names through
include/q38rt_attn.hpp (rope_table -> attn_prep_rows -> attn_prefill for a prefill chunk, then attn_prep_multi ->
attn_decode_multi with the ActQ8 epilogue for a verify block, the order of src/runtime/engine.cpp:2457-2479 and
:1587-1592).  Its outputs must equal the same sequence made through the ctypes mirror bit for bit, and match the
oracle: prep within float rounding, attention within the path's tolerance on the cache as stored."""
import os
import subprocess

import numpy as np
import pytest
import torch

import qwengine_amd.ops as ops
from qwengine_amd.build import SHIM_E2E
from kvutil import KVTS, KV_NAMES, assert_close, dequant_cache

pytestmark = pytest.mark.gpu

THETA, EPS = 1e7, 1e-6


def _inputs(B, nq, seed):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    return dict(qg_pf=f(B, 24, 512), k_pf=f(B, 4, 256), v_pf=f(B, 4, 256),
                qn=(0.5 + rng.random(256)).astype(np.float32), kn=(0.5 + rng.random(256)).astype(np.float32),
                qg_dec=f(nq, 24, 512), k_dec=f(nq, 4, 256), v_dec=f(nq, 4, 256))


def _run_shim(tmp_path, kvt, B, nq, cap, x):
    assert os.path.exists(SHIM_E2E), f"{SHIM_E2E} is not built (python -m qwengine_amd.build)"
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(fin, "wb") as f:
        np.array([kvt, B, nq, cap], np.int32).tofile(f)
        for k in ("qg_pf", "k_pf", "v_pf", "qn", "kn", "qg_dec", "k_dec", "v_dec"):
            x[k].tofile(f)
    print(f"shim_e2e kvt={KV_NAMES[kvt]} B={B} nq={nq}", flush=True)
    r = subprocess.run([SHIM_E2E, str(fin), str(fout)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
    raw = open(fout, "rb").read()
    vb, sb = ops.kv_value_bytes(kvt), ops.kv_scale_bytes(kvt)
    layout = [("out16", np.uint16, B * 6144), ("q_pf", np.float32, B * 6144), ("gate_pf", np.float32, B * 6144),
              ("q_dec", np.float32, nq * 6144), ("gate_dec", np.float32, nq * 6144), ("out", np.float32, nq * 6144),
              ("act_q", np.int8, nq * 6144), ("act_d", np.float32, nq * 192), ("act_s", np.float32, nq * 192),
              ("k", np.uint8, 4 * cap * vb), ("v", np.uint8, 4 * cap * vb)]
    if sb:
        layout += [("ks", np.uint16, 4 * cap * 8), ("vs", np.uint16, 4 * cap * 8)]
    res, off = {}, 0
    for name, dt, n in layout:
        res[name] = np.frombuffer(raw, dt, n, off)
        off += n * np.dtype(dt).itemsize
    assert off == len(raw)
    return res


def _run_ctypes(kvt, B, nq, cap, x):
    t = {k: torch.from_numpy(v).cuda() for k, v in x.items()}
    kv = ops.KVLayer.allocate(kvt, cap)
    rope = torch.empty((B, 64), device="cuda")
    q_pf = torch.empty((B, 24, 256), device="cuda")
    gate_pf = torch.empty_like(q_pf)
    out16 = torch.empty((B, 24, 256), dtype=torch.float16, device="cuda")
    ops.rope_table(0, B, THETA, rope)
    ops.attn_prep_rows(t["qg_pf"], t["k_pf"], t["v_pf"], t["qn"], t["kn"], B, 0, rope, EPS, kvt, kv, q_pf, gate_pf)
    ops.attn_prefill(q_pf, gate_pf, kv, kvt, B, 0, out16)
    q_dec = torch.empty((nq, 24, 256), device="cuda")
    gate_dec = torch.empty_like(q_dec)
    out = torch.empty_like(q_dec)
    act = ops.ActQ8.allocate(nq * 6144)
    work = torch.empty(ops.attn_work_bytes(B + nq) // 4 + 1, dtype=torch.float32, device="cuda")
    ops.attn_prep_multi(ops.RowSrc.device(t["qg_dec"], 12288), ops.RowSrc.device(t["k_dec"], 1024),
                        ops.RowSrc.device(t["v_dec"], 1024), t["qn"], t["kn"], B, B, nq, THETA, EPS, kvt, kv, q_dec,
                        gate_dec)
    ops.attn_decode_multi(q_dec, gate_dec, kv, kvt, B, nq, work, out, act)
    torch.cuda.synchronize()
    return kv, dict(out16=out16.cpu().numpy().view(np.uint16).reshape(-1), q_pf=q_pf.cpu().numpy().reshape(-1),
                    gate_pf=gate_pf.cpu().numpy().reshape(-1), q_dec=q_dec.cpu().numpy().reshape(-1),
                    gate_dec=gate_dec.cpu().numpy().reshape(-1), out=out.cpu().numpy().reshape(-1),
                    act_q=act.q.cpu().numpy().reshape(-1), act_d=act.d.cpu().numpy().reshape(-1),
                    act_s=act.s.cpu().numpy().reshape(-1), k=kv.k.cpu().numpy().reshape(-1),
                    v=kv.v.cpu().numpy().reshape(-1),
                    **({} if kv.ks is None else dict(ks=kv.ks.cpu().numpy().view(np.uint16).reshape(-1),
                                                     vs=kv.vs.cpu().numpy().view(np.uint16).reshape(-1))))


@pytest.mark.parametrize("kvt", KVTS, ids=lambda k: KV_NAMES[k])
def test_shim_prefill_then_verify(gpu, oracle, tmp_path, kvt):
    B, nq, cap = 300, 7, 320
    x = _inputs(B, nq, 900 + kvt)
    got = _run_shim(tmp_path, kvt, B, nq, cap, x)
    kv, want = _run_ctypes(kvt, B, nq, cap, x)
    for name, w in want.items():
        assert np.array_equal(got[name], w), f"{name} differs between the C++ shim and the ctypes path"
    # prep against the double-precision oracle (q within float rounding, gate copied)
    qo, go, _ = oracle.attn_prep_table(x["qg_pf"], x["k_pf"], x["qn"], x["kn"], oracle.rope_table(0, B, THETA), EPS)
    assert np.array_equal(got["gate_pf"].reshape(B, 24, 256), go)
    assert np.abs(got["q_pf"].reshape(B, 24, 256) - qo).max() <= 1e-5 * max(1.0, np.abs(qo).max())
    # attention against the oracle on the cache as the shim stored it
    Kd, Vd = dequant_cache(kv, B + nq)
    pf = oracle.attention(got["q_pf"].reshape(B, 24, 256), got["gate_pf"].reshape(B, 24, 256), Kd, Vd, 0, B)
    assert_close(got["out16"].view(np.float16).astype(np.float32).reshape(B, 24, 256), pf, "shim prefill")
    dec = oracle.attention(got["q_dec"].reshape(nq, 24, 256), got["gate_dec"].reshape(nq, 24, 256), Kd, Vd, B, nq)
    assert_close(got["out"].reshape(nq, 24, 256), dec, "shim verify")
