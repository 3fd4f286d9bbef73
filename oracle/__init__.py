"""CPU oracle for the gated-attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this package, and
only as the checker (or the timed CPU baseline).  The product path in ``qwengine_amd`` never imports it.

numpy front-end over ``oracle/_build/libqwo.so`` (built from ``oracle/qwo.c`` by ``oracle/Makefile``).  Each
function documents the reference lines it restates; see ``oracle/qwo.h`` for the full list.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libqwo.so")
_lib = None

F16, Q8_0, Q4_0 = 0, 1, 2
NH, NKV, D, GROUP = 24, 4, 256, 6

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    args = ["make", "-s", "-C", _HERE]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = ctypes.CDLL(_LIB_PATH)
    L.qwo_fp32_to_fp16.restype = ctypes.c_uint16
    L.qwo_fp32_to_fp16.argtypes = [ctypes.c_float]
    L.qwo_fp16_to_fp32.restype = ctypes.c_float
    L.qwo_fp16_to_fp32.argtypes = [ctypes.c_uint16]
    L.qwo_fp32_to_fp16_n.argtypes = [_f32p, _u16p, _i64]
    L.qwo_fp16_to_fp32_n.argtypes = [_u16p, _f32p, _i64]
    for name in ("qwo_quantize_q8_0", "qwo_quantize_q4_0"):
        getattr(L, name).argtypes = [_f32p, _u8p, _i64]
    for name in ("qwo_dequantize_q8_0", "qwo_dequantize_q4_0"):
        getattr(L, name).argtypes = [_u8p, _f32p, _i64]
    L.qwo_kv_value_bytes.restype = ctypes.c_size_t
    L.qwo_kv_value_bytes.argtypes = [ctypes.c_int]
    L.qwo_kv_scale_bytes.restype = ctypes.c_size_t
    L.qwo_kv_scale_bytes.argtypes = [ctypes.c_int]
    L.qwo_kv_store_rows.argtypes = [ctypes.c_int, _f32p, _i64, _u8p, _u16p]
    L.qwo_kv_load_rows.argtypes = [ctypes.c_int, _u8p, _u16p, _i64, _f32p]
    L.qwo_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                ctypes.c_int, _f32p]
    L.qwo_attn_prep.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                ctypes.c_float, _f32p, _f32p, _f32p]
    L.qwo_attn_prep_table.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_int, _f32p, ctypes.c_float, _f32p, _f32p,
                                      _f32p]
    L.qwo_rope_table.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_float, _f32p]
    L.qwo_rope_table_pos.argtypes = [_i32p, ctypes.c_int, ctypes.c_float, _f32p]
    L.qwo_act_q8.argtypes = [_f32p, _i64, _i8p, _f32p, _f32p]
    L.qwo_max_threads.restype = ctypes.c_int
    L.qwo_deltanet.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, _f32p, _f32p, _f32p, _f32p,
                               ctypes.c_float, _f32p, _f32p, _f32p]
    L.qwo_w_row_bytes.restype = ctypes.c_size_t
    L.qwo_w_row_bytes.argtypes = [ctypes.c_int, _i64]
    L.qwo_iq_grid.restype = ctypes.c_uint64
    L.qwo_iq_grid.argtypes = [ctypes.c_int, ctypes.c_int]
    L.qwo_w_dequant_row.restype = ctypes.c_int
    L.qwo_w_dequant_row.argtypes = [ctypes.c_int, _u8p, _f32p, _i64]
    L.qwo_gemv_ref.restype = ctypes.c_int
    L.qwo_gemv_ref.argtypes = [ctypes.c_int, _u8p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, _i8p, _f32p,
                               ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    _lib = L
    return L


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- fp16 (src/quant/quant_formats.h:29-78) ----
def fp32_to_fp16(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().qwo_fp32_to_fp16_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


def fp16_to_fp32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().qwo_fp16_to_fp32_n(h.reshape(-1), out.reshape(-1), h.size)
    return out


# ---- ggml blocks (src/quant/quant_ref.cpp:302-319,507-538) ----
def quantize_q8_0(x) -> np.ndarray:
    x = _f32(x).reshape(-1)
    out = np.empty(x.size // 32 * 34, np.uint8)
    lib().qwo_quantize_q8_0(x, out, x.size)
    return out


def quantize_q4_0(x) -> np.ndarray:
    x = _f32(x).reshape(-1)
    out = np.empty(x.size // 32 * 18, np.uint8)
    lib().qwo_quantize_q4_0(x, out, x.size)
    return out


def dequantize_q8_0(blocks) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.size // 34 * 32
    out = np.empty(n, np.float32)
    lib().qwo_dequantize_q8_0(blocks, out, n)
    return out


def dequantize_q4_0(blocks) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.size // 18 * 32
    out = np.empty(n, np.float32)
    lib().qwo_dequantize_q4_0(blocks, out, n)
    return out


# ---- split KV layout (src/cuda/ops.cuh:99-113, src/cuda/common.cuh:54-80) ----
def kv_value_bytes(kvt: int) -> int:
    return int(lib().qwo_kv_value_bytes(kvt))


def kv_scale_bytes(kvt: int) -> int:
    return int(lib().qwo_kv_scale_bytes(kvt))


def kv_store_rows(kvt: int, x):
    """x [..., 256] float -> (vals uint8 [..., vb], scales uint16 [..., 8]) in the split layout."""
    x = _f32(x)
    lead = x.shape[:-1]
    n = int(np.prod(lead)) if lead else 1
    vals = np.zeros(lead + (kv_value_bytes(kvt),), np.uint8)
    scales = np.zeros(lead + (8,), np.uint16)
    lib().qwo_kv_store_rows(kvt, x.reshape(-1), n, vals.reshape(-1), scales.reshape(-1))
    return vals, scales


def kv_load_rows(kvt: int, vals, scales) -> np.ndarray:
    vals = np.ascontiguousarray(vals, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    lead = vals.shape[:-1]
    n = int(np.prod(lead)) if lead else 1
    out = np.empty(lead + (256,), np.float32)
    if scales.size == 0:
        scales = np.zeros(8, np.uint16)
    lib().qwo_kv_load_rows(kvt, vals.reshape(-1), scales.reshape(-1), n, out.reshape(-1))
    return out


# ---- attention (src/reference/ref_model.cpp:23-48,138-163) ----
def attention(q, gate, K, V, pos0: int, nq: int, mode: int = 0, threads: int = 0) -> np.ndarray:
    """q, gate [nq,24,256]; K, V dequantized [4, ld, 256] with ld >= pos0+nq.  mode 0 exact, 1 reference arithmetic."""
    q = _f32(q)
    gate = _f32(gate)
    K = _f32(K)
    V = _f32(V)
    assert K.shape == V.shape and K.shape[0] == NKV and K.shape[2] == D and K.shape[1] >= pos0 + nq
    assert q.shape == (nq, NH, D) and gate.shape == (nq, NH, D)
    out = np.empty((nq, NH, D), np.float32)
    lib().qwo_attention(q.reshape(-1), gate.reshape(-1), K.reshape(-1), V.reshape(-1), K.shape[1], pos0, nq, mode,
                        threads, out.reshape(-1))
    return out


# ---- prep (src/cuda/ops.cu:309-358, src/cuda/prefill.cu:344-407) ----
def attn_prep(qg, k, q_norm, k_norm, rope_pos0: int, theta: float, eps: float):
    """qg [n,24,512], k [n,4,256] -> (q [n,24,256], gate [n,24,256], k_roped [n,4,256])."""
    qg = _f32(qg)
    k = _f32(k)
    n = qg.shape[0]
    q_out = np.empty((n, NH, D), np.float32)
    gate = np.empty((n, NH, D), np.float32)
    k_out = np.empty((n, NKV, D), np.float32)
    lib().qwo_attn_prep(qg.reshape(-1), k.reshape(-1), _f32(q_norm), _f32(k_norm), n, rope_pos0, theta, eps,
                        q_out.reshape(-1), gate.reshape(-1), k_out.reshape(-1))
    return q_out, gate, k_out


def attn_prep_table(qg, k, q_norm, k_norm, rope, eps: float):
    qg = _f32(qg)
    k = _f32(k)
    n = qg.shape[0]
    q_out = np.empty((n, NH, D), np.float32)
    gate = np.empty((n, NH, D), np.float32)
    k_out = np.empty((n, NKV, D), np.float32)
    lib().qwo_attn_prep_table(qg.reshape(-1), k.reshape(-1), _f32(q_norm), _f32(k_norm), n, _f32(rope).reshape(-1),
                              eps, q_out.reshape(-1), gate.reshape(-1), k_out.reshape(-1))
    return q_out, gate, k_out


def rope_table(p0: int, B: int, theta: float) -> np.ndarray:
    out = np.empty((B, 64), np.float32)
    lib().qwo_rope_table(p0, B, theta, out.reshape(-1))
    return out


def rope_table_pos(pos, theta: float) -> np.ndarray:
    pos = np.ascontiguousarray(pos, dtype=np.int32).reshape(-1, 3)
    out = np.empty((pos.shape[0], 64), np.float32)
    lib().qwo_rope_table_pos(pos.reshape(-1), pos.shape[0], theta, out.reshape(-1))
    return out


# ---- ActQ8 (src/cuda/common.cuh:188-197) ----
def act_q8(v):
    v = _f32(v).reshape(-1)
    q = np.empty(v.size, np.int8)
    d = np.empty(v.size // 32, np.float32)
    s = np.empty(v.size // 32, np.float32)
    lib().qwo_act_q8(v, v.size, q, d, s)
    return q, d, s


# ---- Gated DeltaNet core (src/reference/ref_model.cpp:169-256) ----
DN_CH, DN_QK, DN_V, DN_VH, DN_KH, DN_HD = 10240, 2048, 6144, 48, 16, 128


def deltanet(qkv, z, b, a, conv_w, dt_bias, ssm_a, ssm_norm, eps, conv_state, S):
    """T tokens of one Gated DeltaNet layer from its projection outputs: qkv [T][10240], z [T][6144], b / a [T][48]
    (raw beta / alpha), conv_w [10240][4], dt_bias / ssm_a [48], ssm_norm [128], conv_state [3][10240] (oldest input
    first), S [48][128 i][128 j] (i = key index).  Returns (o [T][6144], new conv_state, new S); inputs unchanged."""
    qkv = _f32(qkv).reshape(-1, DN_CH)
    T = qkv.shape[0]
    z = _f32(z).reshape(T, DN_V)
    b = _f32(b).reshape(T, -1)
    a = _f32(a).reshape(T, -1)
    assert b.shape == a.shape and b.shape[1] >= DN_VH
    cs = _f32(conv_state).reshape(3, DN_CH).copy()
    St = _f32(S).reshape(DN_VH, DN_HD, DN_HD).copy()
    o = np.empty((T, DN_V), np.float32)
    lib().qwo_deltanet(qkv, z, b, a, b.shape[1], T, _f32(conv_w).reshape(-1), _f32(dt_bias), _f32(ssm_a),
                       _f32(ssm_norm), eps, cs.reshape(-1), St.reshape(-1), o.reshape(-1))
    return o, cs, St


def max_threads() -> int:
    return int(lib().qwo_max_threads())


# ---- weight formats of the output-projection consumer (src/quant/quant_ref.cpp:24-101,281-299) ----
W_Q2_K, W_Q4_K, W_Q6_K, W_IQ4_XS, W_BF16 = 10, 12, 14, 23, 30
# the i-quant grid formats (src/quant/quant_ref.cpp:105-222)
W_IQ2_XXS, W_IQ2_XS, W_IQ3_XXS, W_IQ3_S, W_IQ2_S = 16, 17, 18, 21, 22
IQ_TABLES = {"IQ2XXS": (0, 256, 8), "IQ2XS": (1, 512, 8), "IQ2S": (2, 1024, 8), "IQ3XXS": (3, 256, 4), "IQ3S": (4, 512, 4)}


def iq_grid_bytes(name: str) -> bytes:
    """The expanded byte table of an i-quant codebook (entries little-endian, bytes_per_entry each)."""
    t, n, nb = IQ_TABLES[name]
    return b"".join(int(lib().qwo_iq_grid(t, i)).to_bytes(8, "little")[:nb] for i in range(n))


def w_row_bytes(fmt: int, K: int) -> int:
    return int(lib().qwo_w_row_bytes(fmt, K))


def w_dequant(fmt: int, W, K: int) -> np.ndarray:
    """Rows of ggml-format weights (uint8 [N][row_bytes]) -> fp32 [N][K]."""
    rb = w_row_bytes(fmt, K)
    assert rb > 0
    W = np.ascontiguousarray(W, dtype=np.uint8).reshape(-1, rb)
    out = np.empty((W.shape[0], K), np.float32)
    for r in range(W.shape[0]):
        assert lib().qwo_w_dequant_row(fmt, W[r], out[r], K) == 0
    return out


def gemv_ref(fmt: int, W, K: int, N: int, q, d) -> np.ndarray:
    """float64 y [nc][N] = dequant(W) . (d q) for ActQ8 columns q [nc][K], d [nc][K / 32]."""
    rb = w_row_bytes(fmt, K)
    q = np.ascontiguousarray(q, dtype=np.int8).reshape(-1, K)
    d = _f32(d).reshape(q.shape[0], K // 32)
    y = np.empty((q.shape[0], N), np.float64)
    W = np.ascontiguousarray(W, dtype=np.uint8).reshape(-1)
    assert lib().qwo_gemv_ref(fmt, W, rb, K, N, q.reshape(-1), d.reshape(-1), q.shape[0],
                              y.ctypes.data_as(ctypes.POINTER(ctypes.c_double))) == 0
    return y
