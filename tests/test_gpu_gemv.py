"""GPU parity of the attention output's consumers (src/cuda/gemv.cuh, src/cuda/prefill.cuh:16-18) against the
oracle, with the reference's own criteria (tests/kernels/test_gemv.cu:69-121):

- the decode GEMV within 2e-6 of sum |w| |x| of the float64 product of the dequantized weights and the ActQ8 values;
- the prefill dequantizer bit-exact with the oracle's fp32 value rounded to fp16;
- the activation quantizer bit-exact.

Also: every column of the multi-column GEMV bit-identical to the single-column call, the accumulate flag, the BF16
GEMV, and rejected formats.  Weights are random bytes in each format (no model file ships here); the grid formats
IQ2_XXS / IQ2_XS / IQ2_S / IQ3_XXS / IQ3_S are those of the model's attention output projection."""
import numpy as np
import pytest
import torch

import qwengine_amd.ops as ops
from wutil import random_rows

pytestmark = pytest.mark.gpu

FMTS = [ops.W_Q2_K, ops.W_Q4_K, ops.W_Q6_K, ops.W_IQ4_XS, ops.W_IQ2_XXS, ops.W_IQ2_XS, ops.W_IQ2_S, ops.W_IQ3_XXS,
        ops.W_IQ3_S]
NAMES = {ops.W_Q2_K: "q2_k", ops.W_Q4_K: "q4_k", ops.W_Q6_K: "q6_k", ops.W_IQ4_XS: "iq4_xs", ops.W_BF16: "bf16",
         ops.W_IQ2_XXS: "iq2_xxs", ops.W_IQ2_XS: "iq2_xs", ops.W_IQ2_S: "iq2_s", ops.W_IQ3_XXS: "iq3_xxs",
         ops.W_IQ3_S: "iq3_s"}


def act(x):
    """fp32 rows [n][K] on the GPU -> ActQ8 via the library's quantizer"""
    n, K = x.shape
    a = ops.ActQ8.allocate(n * K)
    ops.quantize_act_q8(x.contiguous(), K, n, a)
    torch.cuda.synchronize()
    return a


def test_quantize_act_q8_bit_exact(gpu, oracle):
    x = torch.randn((3, 5120), device="cuda") * torch.linspace(0.01, 10.0, 5120, device="cuda")
    x[1, :64] = 0.0  # all-zero blocks keep q = 0, d = 0
    a = act(x)
    q, d, s = oracle.act_q8(x.cpu().numpy())
    assert np.array_equal(a.q.cpu().numpy(), q)
    assert np.array_equal(a.d.cpu().numpy().view(np.uint32), d.view(np.uint32))
    assert np.array_equal(a.s.cpu().numpy().view(np.uint32), s.view(np.uint32))


@pytest.mark.parametrize("fmt", FMTS, ids=lambda f: NAMES[f])
@pytest.mark.parametrize("K", [5120, 17408])
def test_gemv_q8_vs_oracle(gpu, oracle, fmt, K):
    print(f"gemv_q8 {NAMES[fmt]} K={K}", flush=True)
    N = 300
    Wn = random_rows(fmt, N, K, 100 + fmt)
    rb = Wn.shape[1]
    W = torch.from_numpy(Wn).cuda()
    x = torch.randn((1, K), device="cuda")
    a = act(x)
    y = torch.empty(N, device="cuda")
    ops.gemv_q8(fmt, W, rb, K, N, a, y)
    torch.cuda.synchronize()
    q, d = a.q.cpu().numpy().reshape(1, K), a.d.cpu().numpy().reshape(1, K // 32)
    ref = oracle.gemv_ref(fmt, Wn, K, N, q, d)[0]
    Wf = oracle.w_dequant(fmt, Wn, K).astype(np.float64)
    xhat = np.repeat(d[0].astype(np.float64), 32) * q[0]
    mag = np.abs(Wf) @ np.abs(xhat)
    err = np.abs(y.cpu().numpy().astype(np.float64) - ref) / mag
    assert err.max() < 2e-6, err.max()


@pytest.mark.parametrize("fmt", FMTS, ids=lambda f: NAMES[f])
def test_gemv_q8n_columns_bitwise_and_accumulate(gpu, fmt):
    K, N = 6144, 257
    Wn = random_rows(fmt, N, K, 200 + fmt)
    rb = Wn.shape[1]
    W = torch.from_numpy(Wn).cuda()
    x = torch.randn((4, K), device="cuda")
    a = act(x)
    singles = []
    for c in range(4):
        ac = ops.ActQ8(a.q[c * K:(c + 1) * K], a.d[c * K // 32:(c + 1) * K // 32], a.s[c * K // 32:(c + 1) * K // 32])
        y = torch.empty(N, device="cuda")
        ops.gemv_q8(fmt, W, rb, K, N, ac, y)
        singles.append(y)
    for nb in range(1, 5):
        y_ld = N + 3
        yn = torch.full((nb, y_ld), float("nan"), device="cuda")
        ops.gemv_q8n(fmt, W, rb, K, N, a, nb, K, yn, y_ld)
        torch.cuda.synchronize()
        for c in range(nb):
            assert torch.equal(yn[c, :N].view(torch.int32), singles[c].view(torch.int32)), (nb, c)
        assert torch.isnan(yn[:, N:]).all()  # padding past N untouched
    base = torch.randn(N, device="cuda")
    y = base.clone()
    ops.gemv_q8(fmt, W, rb, K, N, ops.ActQ8(a.q[:K], a.d[:K // 32], a.s[:K // 32]), y, accumulate=True)
    torch.cuda.synchronize()
    assert torch.equal(y, base + singles[0])


@pytest.mark.parametrize("fmt", FMTS + [ops.W_BF16], ids=lambda f: NAMES[f])
def test_dequant_rows_f16_bit_exact(gpu, oracle, fmt):
    K, rows = 5120, 9
    if fmt == ops.W_BF16:
        Wn = np.random.default_rng(7).standard_normal((rows, K)).astype(np.float32)
        Wn = (Wn.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(rows, 2 * K)
    else:
        Wn = random_rows(fmt, rows, K, 300 + fmt, scale=1.0)
    rb = Wn.shape[1]
    out = torch.empty((rows, K), dtype=torch.float16, device="cuda")
    ops.dequant_rows_f16(fmt, torch.from_numpy(Wn).cuda(), rb, K, rows, out)
    torch.cuda.synchronize()
    want32 = oracle.w_dequant(fmt, Wn, K)
    want = want32.astype(np.float16)  # numpy's fp32 -> fp16 rounds to nearest-even
    got = out.cpu().numpy()
    bad = np.argwhere(got.view(np.uint16) != want.view(np.uint16))
    assert bad.size == 0, [(tuple(i), float(got[tuple(i)]), float(want[tuple(i)]), float(want32[tuple(i)]))
                           for i in bad[:6]]


def test_gemv_bf16(gpu):
    K, N = 5120, 48  # ssm_alpha / ssm_beta shape
    Wf = torch.randn((N, K), device="cuda")
    Wb = (Wf.view(torch.int32) >> 16).to(torch.int16)
    x = torch.randn(K, device="cuda")
    y = torch.empty(N, device="cuda")
    ops.gemv_bf16(Wb.contiguous(), K, N, x, y)
    torch.cuda.synchronize()
    Wd = (Wb.to(torch.int32) << 16).view(torch.float32).double().cpu()
    ref = Wd @ x.double().cpu()
    mag = Wd.abs() @ x.double().cpu().abs()
    assert ((y.double().cpu() - ref).abs() / mag).max() < 1e-6


def test_rejected_formats(gpu):
    W = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    a = ops.ActQ8.allocate(256)
    y = torch.empty(4, device="cuda")
    for fmt in (19, 29, 0):  # IQ1_S, IQ1_M (grid formats without a kernel), FP32
        assert not ops.gemv_q8_supported(fmt)
        with pytest.raises(ops.QwaError):
            ops.gemv_q8(fmt, W, 1024, 256, 4, a, y)
    with pytest.raises(ops.QwaError, match="row_bytes"):
        ops.gemv_q8(ops.W_Q4_K, W, 100, 256, 4, a, y)


@pytest.mark.parametrize("N,K,B,ldx,ldy", [(5120, 6144, 1024, 6144, 5120), (37, 72, 5, 80, 40), (256, 512, 1, 512, 256)])
def test_gemm_f16_vs_float64(gpu, N, K, B, ldx, ldy):
    """Y = X W^T with fp16 inputs and fp32 accumulation (src/cuda/prefill.cuh:20-29) against float64 on the same fp16
    values: within 1e-5 of sum |x| |w|; accumulate adds onto Y; columns past N in a padded Y row stay untouched."""
    print(f"gemm_f16 N={N} K={K} B={B}", flush=True)
    g = ops.Gemm()
    W = (torch.randn((N, K), device="cuda") * 0.05).half()
    X = torch.randn((B, ldx), device="cuda").half()
    Y = torch.full((B, ldy), float("nan"), device="cuda")
    g.f16(W, N, K, X, ldx, B, Y, ldy)
    torch.cuda.synchronize()
    Xd, Wd = X[:, :K].double(), W.double()
    ref = Xd @ Wd.T
    mag = Xd.abs() @ Wd.abs().T
    assert ((Y[:, :N].double() - ref).abs() / mag).max().item() < 1e-5
    if ldy > N:
        assert torch.isnan(Y[:, N:]).all()
    Y0 = Y.clone()
    g.f16(W, N, K, X, ldx, B, Y, ldy, accumulate=True)
    torch.cuda.synchronize()
    assert ((Y[:, :N].double() - 2 * ref).abs() / mag).max().item() < 2e-5
    assert torch.allclose(Y[:, :N], 2 * Y0[:, :N], rtol=1e-6, atol=1e-6)
    g.close()


def test_gemm_tune_keeps_a_correct_algorithm(gpu):
    """qwa_gemm_tune times hipBLASLt's candidates for a shape and keeps the fastest: later calls of the shape stay
    within the same float64 bound, and tuning is refused while the stream is capturing."""
    N, K, B = 640, 1024, 96
    g = ops.Gemm()
    W = (torch.randn((N, K), device="cuda") * 0.05).half()
    X = torch.randn((B, K), device="cuda").half()
    Y = torch.empty((B, N), device="cuda")
    us = g.tune(W, N, K, X, K, B, Y, N, max_candidates=8)
    assert us > 0.0
    Y.fill_(float("nan"))
    g.f16(W, N, K, X, K, B, Y, N)
    torch.cuda.synchronize()
    Xd, Wd = X.double(), W.double()
    assert ((Y.double() - Xd @ Wd.T).abs() / (Xd.abs() @ Wd.abs().T)).max().item() < 1e-5
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        with pytest.raises(ops.QwaError):
            g.tune(W, N, K, X, K, B, Y, N, stream=s)
    g.close()

