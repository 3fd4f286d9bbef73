"""Host-side mirror of the reference's attention / KV-cache operators, over the C ABI of ``libqwattn.so``.

Names, argument meaning and error behaviour follow ``q38rt::cuda`` (src/cuda/ops.cuh:99-140,
src/cuda/prefill.cuh:46-62): buffers are caller-owned device tensors, every call is asynchronous on the current
HIP stream (or ``stream=``), nothing is allocated by an operator, and an invalid call raises ``QwaError`` where the
reference aborts.  torch is used only for device memory and streams.

The HIP library must be built (``python -m qwengine_amd.build``); calls fail loudly when it is missing -- there is
no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

F16, Q8_0, Q4_0 = 0, 1, 2
KV_TYPES = {"f16": F16, "q8_0": Q8_0, "q4_0": Q4_0}
N_HEAD, N_KV, HEAD_DIM, GROUP = 24, 4, 256, 6

# QWA_LIBRARY selects another build of the same library (e.g. one compiled with different tuning macros)
_LIB_PATH = os.environ.get("QWA_LIBRARY") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib",
                                                          "libqwattn.so")
_lib = None


class QwaError(RuntimeError):
    """An operator rejected its arguments or a launch failed (the reference aborts in these cases)."""


class _KVLayerC(ctypes.Structure):
    _fields_ = [("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("ks", ctypes.c_void_p), ("vs", ctypes.c_void_p),
                ("capacity", ctypes.c_int)]


class _ActQ8C(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("d", ctypes.c_void_p), ("s", ctypes.c_void_p)]


class _RowSrcC(ctypes.Structure):
    _fields_ = [("dev", ctypes.c_void_p), ("host", ctypes.c_void_p), ("split", ctypes.c_int), ("host_ld", ctypes.c_int)]


class _DNParamsC(ctypes.Structure):
    _fields_ = [("conv_w", ctypes.c_void_p), ("dt_bias", ctypes.c_void_p), ("ssm_a", ctypes.c_void_p),
                ("ssm_norm", ctypes.c_void_p), ("conv_state", ctypes.c_void_p), ("ssm_state", ctypes.c_void_p)]


class _DNTokensC(ctypes.Structure):
    _fields_ = [("sqkv", ctypes.c_void_p), ("sbeta", ctypes.c_void_p), ("salpha", ctypes.c_void_p),
                ("qkv", ctypes.c_void_p), ("z", ctypes.c_void_p), ("beta", ctypes.c_void_p), ("alpha", ctypes.c_void_p),
                ("oqkv", ctypes.c_void_p), ("obeta", ctypes.c_void_p), ("oalpha", ctypes.c_void_p),
                ("qkv_host", ctypes.c_void_p), ("qkv_split", ctypes.c_int), ("qkv_ld", ctypes.c_int),
                ("z_host", ctypes.c_void_p), ("z_split", ctypes.c_int), ("z_ld", ctypes.c_int),
                ("o_host", ctypes.c_void_p)]


EXPORTS = {
    # name: (restype, argtypes)
    "qwa_kv_value_bytes": (ctypes.c_size_t, [ctypes.c_int]),
    "qwa_kv_scale_bytes": (ctypes.c_size_t, [ctypes.c_int]),
    "qwa_attn_prep": (ctypes.c_int, [ctypes.c_void_p] * 5 + [ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int,
                                                             ctypes.POINTER(_KVLayerC), ctypes.c_void_p,
                                                             ctypes.c_void_p, ctypes.c_void_p]),
    "qwa_attn_prep_multi": (ctypes.c_int, [ctypes.POINTER(_RowSrcC)] * 3 + [ctypes.c_void_p] * 2 +
                            [ctypes.c_int] * 3 + [ctypes.c_float] * 2 + [ctypes.c_int, ctypes.POINTER(_KVLayerC)] +
                            [ctypes.c_void_p] * 3),
    "qwa_attn_work_bytes": (ctypes.c_size_t, [ctypes.c_int]),
    "qwa_attn_max_positions": (ctypes.c_int, []),
    "qwa_attn_decode": (ctypes.c_int, [ctypes.c_void_p] * 2 + [ctypes.POINTER(_KVLayerC), ctypes.c_int, ctypes.c_int,
                                                               ctypes.c_void_p, ctypes.c_void_p,
                                                               ctypes.POINTER(_ActQ8C), ctypes.c_void_p]),
    "qwa_attn_decode_multi": (ctypes.c_int, [ctypes.c_void_p] * 2 + [ctypes.POINTER(_KVLayerC)] + [ctypes.c_int] * 3 +
                              [ctypes.c_void_p] * 2 + [ctypes.POINTER(_ActQ8C), ctypes.c_void_p, ctypes.c_void_p]),
    "qwa_attn_decode_multi_noalloc": (ctypes.c_int, [ctypes.c_void_p] * 2 + [ctypes.POINTER(_KVLayerC)] +
                                      [ctypes.c_int] * 3 + [ctypes.c_void_p, ctypes.POINTER(_ActQ8C), ctypes.c_void_p,
                                                            ctypes.c_void_p]),
    "qwa_attn_decode_simple": (ctypes.c_int, [ctypes.c_void_p] * 2 + [ctypes.POINTER(_KVLayerC), ctypes.c_int,
                                                                      ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                                                      ctypes.POINTER(_ActQ8C), ctypes.c_void_p]),
    "qwa_rope_table": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p]),
    "qwa_rope_table_pos": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_void_p,
                                          ctypes.c_void_p]),
    "qwa_attn_prep_rows": (ctypes.c_int, [ctypes.c_void_p] * 5 + [ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                                                  ctypes.c_float, ctypes.c_int,
                                                                  ctypes.POINTER(_KVLayerC)] + [ctypes.c_void_p] * 3),
    "qwa_attn_prefill": (ctypes.c_int, [ctypes.c_void_p] * 2 + [ctypes.POINTER(_KVLayerC)] + [ctypes.c_int] * 3 +
                         [ctypes.c_void_p] * 2),
    "qwa_attn_prefill_reserve": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "qwa_attn_prefill_release": (ctypes.c_int, [ctypes.c_void_p]),
    "qwa_attn_prefill_work_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int]),
    "qwa_attn_prefill_ws": (ctypes.c_int, [ctypes.c_void_p] * 2 + [ctypes.POINTER(_KVLayerC)] + [ctypes.c_int] * 3 +
                            [ctypes.c_void_p] * 2 + [ctypes.c_size_t, ctypes.c_void_p]),
    "qwa_attn_prefill_simple": (ctypes.c_int, [ctypes.c_void_p] * 2 + [ctypes.POINTER(_KVLayerC)] +
                                [ctypes.c_int] * 3 + [ctypes.c_void_p] * 2),
    "qwa_kv_append": (ctypes.c_int, [ctypes.c_void_p] * 2 + [ctypes.c_int] * 3 + [ctypes.POINTER(_KVLayerC),
                                                                                  ctypes.c_void_p]),
    "qwa_kv_packed_bytes": (ctypes.c_longlong, [ctypes.c_int, ctypes.c_int]),
    "qwa_kv_pack": (ctypes.c_int, [ctypes.POINTER(_KVLayerC), ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                   ctypes.c_void_p]),
    "qwa_kv_unpack": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(_KVLayerC), ctypes.c_int, ctypes.c_int,
                                     ctypes.c_void_p]),
    "qwa_deltanet_step": (ctypes.c_int, [ctypes.POINTER(_DNParamsC)] + [ctypes.c_void_p] * 4 +
                          [ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.POINTER(_ActQ8C), ctypes.c_void_p]),
    "qwa_deltanet_multi": (ctypes.c_int, [ctypes.POINTER(_DNParamsC), ctypes.c_int, ctypes.POINTER(_DNTokensC)] +
                           [ctypes.c_int] * 3 + [ctypes.c_float, ctypes.c_void_p, ctypes.POINTER(_ActQ8C),
                                                 ctypes.c_void_p]),
    "qwa_dn_work_bytes": (ctypes.c_size_t, [ctypes.c_int]),
    "qwa_w_row_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_longlong]),
    "qwa_gemm_create": (ctypes.c_void_p, []),
    "qwa_gemm_bind": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]),
    "qwa_gemm_destroy": (None, [ctypes.c_void_p]),
    "qwa_gemm_f16": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p]),
    "qwa_gemm_tune": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)]),
    "qwa_gemv_q8_supported": (ctypes.c_int, [ctypes.c_int]),
    "qwa_quantize_act_q8": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_ActQ8C),
                                           ctypes.c_void_p]),
    "qwa_gemv_q8": (ctypes.c_int, [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                   ctypes.POINTER(_ActQ8C), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]),
    "qwa_gemv_q8n": (ctypes.c_int, [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                    ctypes.POINTER(_ActQ8C), ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                    ctypes.c_int, ctypes.c_void_p, ctypes.c_int]),
    "qwa_gemv_bf16": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_void_p]),
    "qwa_dequant_rows_f16": (ctypes.c_int, [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]),
    "qwa_deltanet_rows": (ctypes.c_int, [ctypes.POINTER(_DNParamsC)] + [ctypes.c_void_p] * 4 +
                          [ctypes.c_int, ctypes.c_int, ctypes.c_float] + [ctypes.c_void_p] * 4),
    "qwa_profile_begin": (ctypes.c_int, []),
    "qwa_profile_end": (ctypes.c_int, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int)]),
    "qwa_profile_device_ms": (ctypes.c_int, [ctypes.POINTER(ctypes.c_double)]),
    "qwa_profile_clock_mhz": (ctypes.c_int, [ctypes.POINTER(ctypes.c_double)]),
    "qwa_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "qwa_last_error": (ctypes.c_char_p, []),
}


def library_path() -> str:
    return _LIB_PATH


def lib():
    """Load libqwattn.so (raises if it has not been built: there is no fallback path)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise QwaError(f"HIP library missing: {_LIB_PATH} (build it with `python -m qwengine_amd.build`)")
        L = ctypes.CDLL(_LIB_PATH)
        for name, (res, args) in EXPORTS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(status: int) -> None:
    if status != 0:
        L = lib()
        raise QwaError(f"{L.qwa_status_string(status).decode()}: {L.qwa_last_error().decode()}")


def _ptr(t) -> int | None:
    if t is None:
        return None
    if not isinstance(t, torch.Tensor):
        return int(t)
    if not t.is_contiguous():
        raise QwaError("tensor arguments must be contiguous")
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream if torch.cuda.is_available() else None
    if isinstance(stream, torch.cuda.Stream):
        return stream.cuda_stream
    return int(stream)


def _kvt(kvt) -> int:
    return KV_TYPES[kvt] if isinstance(kvt, str) else int(kvt)


def kv_value_bytes(kvt) -> int:
    """Bytes of one 256-value head row (src/cuda/ops.cu:966-973)."""
    return int(lib().qwa_kv_value_bytes(_kvt(kvt)))


def kv_scale_bytes(kvt) -> int:
    """Bytes of one row's fp16 block scales (src/cuda/ops.cu:974)."""
    return int(lib().qwa_kv_scale_bytes(_kvt(kvt)))


@dataclass
class KVLayer:
    """Per-layer KV cache in the split layout (mirror of q38rt::cuda::KVLayer, src/cuda/ops.cuh:106-113).

    k, v: uint8 [4, capacity, value_bytes]; ks, vs: int16 [4, capacity, 8] fp16 bits (None for F16)."""
    kvt: int
    capacity: int
    k: torch.Tensor
    v: torch.Tensor
    ks: torch.Tensor | None
    vs: torch.Tensor | None

    @classmethod
    def allocate(cls, kvt, capacity: int, device="cuda", zero: bool = True) -> "KVLayer":
        kvt = _kvt(kvt)
        vb = kv_value_bytes(kvt)
        alloc = torch.zeros if zero else torch.empty
        k = alloc((N_KV, capacity, vb), dtype=torch.uint8, device=device)
        v = alloc((N_KV, capacity, vb), dtype=torch.uint8, device=device)
        ks = vs = None
        if kvt != F16:
            ks = alloc((N_KV, capacity, 8), dtype=torch.int16, device=device)
            vs = alloc((N_KV, capacity, 8), dtype=torch.int16, device=device)
        return cls(kvt, capacity, k, v, ks, vs)

    def c(self) -> _KVLayerC:
        return _KVLayerC(_ptr(self.k), _ptr(self.v), _ptr(self.ks), _ptr(self.vs), self.capacity)

    def nbytes(self) -> int:
        n = self.k.numel() + self.v.numel()
        if self.ks is not None:
            n += 2 * (self.ks.numel() + self.vs.numel())
        return n


@dataclass
class ActQ8:
    """int8 activations with per-32 scales (mirror of q38rt::cuda::ActQ8, src/cuda/gemv.cuh:14-18)."""
    q: torch.Tensor
    d: torch.Tensor
    s: torch.Tensor

    @classmethod
    def allocate(cls, n: int, device="cuda") -> "ActQ8":
        return cls(torch.empty(n, dtype=torch.int8, device=device), torch.empty(n // 32, dtype=torch.float32,
                                                                                   device=device),
                   torch.empty(n // 32, dtype=torch.float32, device=device))

    def c(self) -> _ActQ8C:
        return _ActQ8C(_ptr(self.q), _ptr(self.d), _ptr(self.s))


@dataclass
class RowSrc:
    """Row source with a device head and an optional mapped-host tail (mirror of RowSrc, src/cuda/ops.cuh:24-34)."""
    dev: object
    split: int
    host: object = None
    host_ld: int = 0

    @classmethod
    def device(cls, t, n: int) -> "RowSrc":
        return cls(t, n)

    def c(self) -> _RowSrcC:
        return _RowSrcC(_ptr(self.dev), _ptr(self.host), self.split, self.host_ld)


def _act(oq):
    return ctypes.byref(oq.c()) if oq is not None else None


def attn_prep(qg, k, v, q_norm, k_norm, pos: int, theta: float, eps: float, kvt, kv: KVLayer, q_out, gate,
              stream=None) -> None:
    """src/cuda/ops.cuh:117-118."""
    _check(lib().qwa_attn_prep(_ptr(qg), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm), pos, theta, eps, _kvt(kvt),
                               ctypes.byref(kv.c()), _ptr(q_out), _ptr(gate), _stream(stream)))


def attn_prep_multi(qg: RowSrc, k: RowSrc, v: RowSrc, q_norm, k_norm, pos0: int, rope_pos0: int, n: int,
                    theta: float, eps: float, kvt, kv: KVLayer, q_out, gate, stream=None) -> None:
    """src/cuda/ops.cuh:122-124."""
    _check(lib().qwa_attn_prep_multi(ctypes.byref(qg.c()), ctypes.byref(k.c()), ctypes.byref(v.c()), _ptr(q_norm),
                                     _ptr(k_norm), pos0, rope_pos0, n, theta, eps, _kvt(kvt), ctypes.byref(kv.c()),
                                     _ptr(q_out), _ptr(gate), _stream(stream)))


def attn_work_bytes(n_pos: int) -> int:
    """src/cuda/ops.cuh:129."""
    return int(lib().qwa_attn_work_bytes(n_pos))


def attn_max_positions() -> int:
    """src/cuda/ops.cuh:131."""
    return int(lib().qwa_attn_max_positions())


def attn_decode(q, gate, kv: KVLayer, kvt, n_pos: int, work, out, oq: ActQ8 | None = None, stream=None) -> None:
    """src/cuda/ops.cuh:132-133."""
    _check(lib().qwa_attn_decode(_ptr(q), _ptr(gate), ctypes.byref(kv.c()), _kvt(kvt), n_pos, _ptr(work), _ptr(out),
                                 _act(oq), _stream(stream)))


def attn_decode_multi(q, gate, kv: KVLayer, kvt, pos0: int, nq: int, work, out, oq: ActQ8 | None = None,
                      stream=None, out_host=None) -> None:
    """src/cuda/ops.cuh:136-137."""
    _check(lib().qwa_attn_decode_multi(_ptr(q), _ptr(gate), ctypes.byref(kv.c()), _kvt(kvt), pos0, nq, _ptr(work),
                                       _ptr(out), _act(oq), _stream(stream), _ptr(out_host)))


def attn_decode_multi_noalloc(q, gate, kv: KVLayer, kvt, pos0: int, nq: int, out, oq: ActQ8 | None = None,
                              stream=None, out_host=None) -> None:
    """attn_decode_multi on the library's static scratch: no work argument, nothing allocated (no reference
    counterpart).  Calls that overlap on one GPU race on that scratch."""
    _check(lib().qwa_attn_decode_multi_noalloc(_ptr(q), _ptr(gate), ctypes.byref(kv.c()), _kvt(kvt), pos0, nq,
                                               _ptr(out), _act(oq), _stream(stream), _ptr(out_host)))


def attn_decode_simple(q, gate, kv: KVLayer, kvt, n_pos: int, work, out, oq: ActQ8 | None = None,
                       stream=None) -> None:
    """src/cuda/ops.cuh:139-140."""
    _check(lib().qwa_attn_decode_simple(_ptr(q), _ptr(gate), ctypes.byref(kv.c()), _kvt(kvt), n_pos, _ptr(work),
                                        _ptr(out), _act(oq), _stream(stream)))


def rope_table(p0: int, B: int, theta: float, rope, stream=None) -> None:
    """src/cuda/prefill.cuh:46-48."""
    _check(lib().qwa_rope_table(p0, B, theta, _ptr(rope), _stream(stream)))


def rope_table_pos(pos, B: int, theta: float, rope, stream=None) -> None:
    """src/cuda/prefill.cuh:49-52."""
    _check(lib().qwa_rope_table_pos(_ptr(pos), B, theta, _ptr(rope), _stream(stream)))


def attn_prep_rows(qg, k, v, q_norm, k_norm, B: int, p0: int, rope, eps: float, kvt, kv: KVLayer, q, gate,
                   stream=None) -> None:
    """src/cuda/prefill.cuh:55-56."""
    _check(lib().qwa_attn_prep_rows(_ptr(qg), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm), B, p0, _ptr(rope), eps,
                                    _kvt(kvt), ctypes.byref(kv.c()), _ptr(q), _ptr(gate), _stream(stream)))


def attn_prefill(q, gate, kv: KVLayer, kvt, B: int, p0: int, out16, stream=None) -> None:
    """src/cuda/prefill.cuh:59-60 (out16: fp16 [B, 6144]).  Uses the stream's prefill workspace; a call it does not
    cover widens it first (allocates), except under graph capture, where it raises QwaError."""
    _check(lib().qwa_attn_prefill(_ptr(q), _ptr(gate), ctypes.byref(kv.c()), _kvt(kvt), B, p0, _ptr(out16),
                                  _stream(stream)))


def attn_prefill_reserve(max_B: int, max_pos: int, stream=None) -> None:
    """Set-up: reserve the prefill workspace of the stream (calls with B <= max_B, p0 + B <= max_pos)."""
    _check(lib().qwa_attn_prefill_reserve(max_B, max_pos, _stream(stream)))


def attn_prefill_release(stream=None) -> None:
    _check(lib().qwa_attn_prefill_release(_stream(stream)))


def attn_prefill_work_bytes(B: int, n_pos: int) -> int:
    return int(lib().qwa_attn_prefill_work_bytes(B, n_pos))


def attn_prefill_ws(q, gate, kv: KVLayer, kvt, B: int, p0: int, out16, work, stream=None) -> None:
    """attn_prefill with a caller-owned workspace tensor of at least attn_prefill_work_bytes(B, p0 + B) bytes."""
    _check(lib().qwa_attn_prefill_ws(_ptr(q), _ptr(gate), ctypes.byref(kv.c()), _kvt(kvt), B, p0, _ptr(out16),
                                     _ptr(work), work.numel() * work.element_size(), _stream(stream)))


def attn_prefill_simple(q, gate, kv: KVLayer, kvt, B: int, p0: int, out16, stream=None) -> None:
    """src/cuda/prefill.cuh:61-62."""
    _check(lib().qwa_attn_prefill_simple(_ptr(q), _ptr(gate), ctypes.byref(kv.c()), _kvt(kvt), B, p0, _ptr(out16),
                                         _stream(stream)))


def profile_begin() -> None:
    """Start timing the main kernel of every attention call (HIP events around each launch)."""
    _check(lib().qwa_profile_begin())


def profile_end() -> tuple[float, int]:
    """Stop timing; returns (summed main-kernel time in ms from the HIP events around each launch, number of timed
    launches)."""
    ms = ctypes.c_double(0.0)
    n = ctypes.c_int(0)
    _check(lib().qwa_profile_end(ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value


def profile_device_ms() -> float:
    """Summed device-clock time of the last closed window (first workgroup start to last workgroup end per launch)."""
    ms = ctypes.c_double(0.0)
    _check(lib().qwa_profile_device_ms(ctypes.byref(ms)))
    return ms.value


def profile_clock_mhz() -> float:
    """Shader clock (MHz) the last closed window's workgroups ran at: shader-clock ticks over realtime ticks, summed
    over every workgroup's lifetime."""
    mhz = ctypes.c_double(0.0)
    _check(lib().qwa_profile_clock_mhz(ctypes.byref(mhz)))
    return mhz.value


def kv_packed_bytes(kvt, n_pos: int) -> int:
    """Bytes of the packed (parked) form of the first n_pos positions of a layer (the engine's resize layout)."""
    return int(lib().qwa_kv_packed_bytes(_kvt(kvt), n_pos))


def kv_pack(kv: KVLayer, kvt, n_pos: int, dst, stream=None) -> None:
    """Copies positions [0, n_pos) of every KV head into dst (device tensor or pinned host tensor), packed."""
    _check(lib().qwa_kv_pack(ctypes.byref(kv.c()), _kvt(kvt), n_pos, _ptr(dst), _stream(stream)))


def kv_unpack(src, kv: KVLayer, kvt, n_pos: int, stream=None) -> None:
    """Restores a packed prefix into positions [0, n_pos) of a layer of any capacity >= n_pos."""
    _check(lib().qwa_kv_unpack(_ptr(src), ctypes.byref(kv.c()), _kvt(kvt), n_pos, _stream(stream)))


def kv_append(xk, xv, pos0: int, n: int, kvt, kv: KVLayer, stream=None) -> None:
    """Quantize-on-append of raw K/V rows [n, 4, 256] (the row store of src/cuda/common.cuh:54-80)."""
    _check(lib().qwa_kv_append(_ptr(xk), _ptr(xv), pos0, n, _kvt(kvt), ctypes.byref(kv.c()), _stream(stream)))


# ---- Gated DeltaNet ------------------------------------------------------------------------------------------------
DN_CH, DN_QK, DN_VD, DN_VH, DN_KH, DN_HD, DN_MAXN = 10240, 2048, 6144, 48, 16, 128, 7


@dataclass
class DNParams:
    """One Gated DeltaNet layer (mirror of q38rt::cuda::DeltaNetParams, src/cuda/ops.cuh:54-62).

    conv_w [10240][4], dt_bias / ssm_a [48], ssm_norm [128] fp32; conv_state [2][3][10240] (ping-pong buffers);
    ssm_state [48][128 col j][128 row i] fp32."""
    conv_w: torch.Tensor
    dt_bias: torch.Tensor
    ssm_a: torch.Tensor
    ssm_norm: torch.Tensor
    conv_state: torch.Tensor
    ssm_state: torch.Tensor

    def c(self) -> _DNParamsC:
        return _DNParamsC(_ptr(self.conv_w), _ptr(self.dt_bias), _ptr(self.ssm_a), _ptr(self.ssm_norm),
                          _ptr(self.conv_state), _ptr(self.ssm_state))


@dataclass
class DNTokens:
    """Token inputs of deltanet_multi (mirror of q38rt::cuda::DNTokens, src/cuda/ops.cuh:74-91).  Host parts:
    qkv channels >= qkv_split come from qkv_host [n][qkv_ld], z channels >= z_split from z_host [n][z_ld]."""
    sqkv: object = None
    sbeta: object = None
    salpha: object = None
    qkv: object = None
    z: object = None
    beta: object = None
    alpha: object = None
    oqkv: object = None
    obeta: object = None
    oalpha: object = None
    qkv_host: object = None
    qkv_split: int = 1 << 30
    qkv_ld: int = 0
    z_host: object = None
    z_split: int = 1 << 30
    z_ld: int = 0
    o_host: object = None

    def c(self) -> _DNTokensC:
        return _DNTokensC(_ptr(self.sqkv), _ptr(self.sbeta), _ptr(self.salpha), _ptr(self.qkv), _ptr(self.z),
                          _ptr(self.beta), _ptr(self.alpha), _ptr(self.oqkv), _ptr(self.obeta), _ptr(self.oalpha),
                          _ptr(self.qkv_host), self.qkv_split, self.qkv_ld, _ptr(self.z_host), self.z_split,
                          self.z_ld, _ptr(self.o_host))


def deltanet_step(p: DNParams, qkv, z, beta_raw, alpha_raw, parity: int, eps: float, o, oq: ActQ8 | None = None,
                  stream=None) -> None:
    """src/cuda/ops.cuh:67-68."""
    _check(lib().qwa_deltanet_step(ctypes.byref(p.c()), _ptr(qkv), _ptr(z), _ptr(beta_raw), _ptr(alpha_raw), parity,
                                   eps, _ptr(o), _act(oq), _stream(stream)))


def deltanet_multi(p: DNParams, cin: int, tokens: DNTokens, n_commit: int, n_new: int, write_after: int, eps: float,
                   o, oq: ActQ8 | None = None, stream=None) -> None:
    """src/cuda/ops.cuh:96-97."""
    _check(lib().qwa_deltanet_multi(ctypes.byref(p.c()), cin, ctypes.byref(tokens.c()), n_commit, n_new,
                                    write_after, eps, _ptr(o), _act(oq), _stream(stream)))


def dn_work_bytes(B: int) -> int:
    """src/cuda/prefill.cuh:41."""
    return int(lib().qwa_dn_work_bytes(B))


def deltanet_rows(p: DNParams, qkv, z, beta_raw, alpha_raw, B: int, cin: int, eps: float, work, core_out, o16,
                  stream=None) -> None:
    """src/cuda/prefill.cuh:42-44."""
    _check(lib().qwa_deltanet_rows(ctypes.byref(p.c()), _ptr(qkv), _ptr(z), _ptr(beta_raw), _ptr(alpha_raw), B, cin,
                                   eps, _ptr(work), _ptr(core_out), _ptr(o16), _stream(stream)))


# ---- consumers of the attention output (src/cuda/gemv.cuh:20-39, src/cuda/prefill.cuh:16-18) ------------------------
W_Q2_K, W_Q4_K, W_Q6_K, W_IQ4_XS, W_BF16 = 10, 12, 14, 23, 30
W_IQ2_XXS, W_IQ2_XS, W_IQ3_XXS, W_IQ3_S, W_IQ2_S = 16, 17, 18, 21, 22


def w_row_bytes(fmt: int, K: int) -> int:
    return int(lib().qwa_w_row_bytes(fmt, K))


def gemv_q8_supported(fmt: int) -> bool:
    return bool(lib().qwa_gemv_q8_supported(fmt))


def quantize_act_q8(x, K: int, n_rows: int, out: ActQ8, stream=None) -> None:
    """src/cuda/gemv.cuh:20-21."""
    _check(lib().qwa_quantize_act_q8(_ptr(x), K, n_rows, ctypes.byref(out.c()), _stream(stream)))


def gemv_q8(fmt: int, W, row_bytes: int, K: int, N: int, act: ActQ8, y, stream=None, accumulate=False) -> None:
    """src/cuda/gemv.cuh:23-27."""
    _check(lib().qwa_gemv_q8(fmt, _ptr(W), row_bytes, K, N, ctypes.byref(act.c()), _ptr(y), _stream(stream),
                             1 if accumulate else 0))


def gemv_q8n(fmt: int, W, row_bytes: int, K: int, N: int, act: ActQ8, nb: int, act_ld: int, y, y_ld: int,
             stream=None, accumulate=False) -> None:
    """src/cuda/gemv.cuh:33-36."""
    _check(lib().qwa_gemv_q8n(fmt, _ptr(W), row_bytes, K, N, ctypes.byref(act.c()), nb, act_ld, _ptr(y), y_ld,
                              _stream(stream), 1 if accumulate else 0))


def gemv_bf16(W, K: int, N: int, x, y, stream=None) -> None:
    """src/cuda/gemv.cuh:29-30."""
    _check(lib().qwa_gemv_bf16(_ptr(W), K, N, _ptr(x), _ptr(y), _stream(stream)))


def dequant_rows_f16(fmt: int, W, row_bytes: int, K: int, rows: int, out, stream=None) -> None:
    """src/cuda/prefill.cuh:16-18."""
    _check(lib().qwa_dequant_rows_f16(fmt, _ptr(W), row_bytes, K, rows, _ptr(out), _stream(stream)))


class Gemm:
    """hipBLASLt FP16 GEMM handle (mirror of cublas_create / cublas_bind / gemm_f16, src/cuda/prefill.cuh:20-29)."""

    def __init__(self, workspace_bytes: int = 32 << 20, stream=None):
        self.h = lib().qwa_gemm_create()
        if not self.h:
            raise QwaError("hipBLASLt could not be initialised")
        self.ws = torch.empty(max(workspace_bytes, 1), dtype=torch.uint8, device="cuda")
        _check(lib().qwa_gemm_bind(self.h, _stream(stream), _ptr(self.ws), workspace_bytes))

    def f16(self, W, N: int, K: int, X, ldx: int, B: int, Y, ldy: int, accumulate=False, stream=None) -> None:
        _check(lib().qwa_gemm_f16(self.h, _ptr(W), N, K, _ptr(X), ldx, B, _ptr(Y), ldy, 1 if accumulate else 0,
                                  _stream(stream)))

    def tune(self, W, N: int, K: int, X, ldx: int, B: int, Y, ldy: int, max_candidates: int = 16,
             stream=None) -> float:
        """Times hipBLASLt's first candidates for this shape (Y is overwritten) and keeps the fastest; returns its
        time per call in microseconds.  Set-up only: refused while the stream captures."""
        best = ctypes.c_float(0.0)
        _check(lib().qwa_gemm_tune(self.h, _ptr(W), N, K, _ptr(X), ldx, B, _ptr(Y), ldy, max_candidates,
                                   _stream(stream), ctypes.byref(best)))
        return best.value

    def close(self) -> None:
        if self.h:
            lib().qwa_gemm_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
