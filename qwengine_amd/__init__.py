"""qwengine_amd: MI355X (gfx950) gated-attention hot path of QWENgine -- decode, speculative verify and prefill
attention over the F16 / Q8_0 / Q4_0 KV cache with fused sigmoid gate and quantize-on-append.

The kernels are hand-written HIP in ``qwengine_amd/csrc`` behind the C ABI ``include/qwattn.h``;
``qwengine_amd.ops`` mirrors the reference's ``q38rt::cuda`` operator interface on top of it.
"""
from . import ops  # noqa: F401
from .ops import (ActQ8, KVLayer, QwaError, RowSrc, F16, Q8_0, Q4_0)  # noqa: F401

__all__ = ["ops", "ActQ8", "KVLayer", "QwaError", "RowSrc", "F16", "Q8_0", "Q4_0"]
