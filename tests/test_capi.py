"""The C ABI library (no GPU needed): it loads, exports every entry point include/qwattn.h declares, answers the
host-only queries, and rejects invalid calls before launching anything (the reference aborts on the same inputs,
src/cuda/ops.cu:1002-1008).  The C++ shim include/q38rt_attn.hpp compiles against it with the reference's names."""
import ctypes
import os
import re
import subprocess

import pytest

import qwengine_amd.ops as ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qwattn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qwa_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 17
    lib = ctypes.CDLL(ops.library_path())
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python mirror binds exactly those
    assert sorted(ops.EXPORTS) == names


def test_host_queries():
    assert ops.kv_value_bytes("f16") == 512
    assert ops.kv_value_bytes("q8_0") == 256
    assert ops.kv_value_bytes("q4_0") == 128
    assert ops.kv_value_bytes(7) == 0
    assert ops.kv_scale_bytes("f16") == 0 and ops.kv_scale_bytes("q4_0") == 16
    assert ops.attn_max_positions() == 262144
    # the work buffer holds one partial record (m, l, O[256]) per decode workgroup, KV head, query (<= 8) and head
    w = ops.attn_work_bytes(150000)
    assert w >= 128 * 4 * 8 * 6 * 258 * 4  # 128 record slots per KV head
    assert ops.attn_work_bytes(1) > 0


class _Fake:
    """A non-null 'device pointer' that is never dereferenced: every call below is rejected on the host."""

    def __init__(self, v=0x1000):
        self.v = v


def _kv(kvt, cap=1024):
    p = 0x10000
    return ops.KVLayer(ops._kvt(kvt), cap, p, p, None if kvt == "f16" else p, None if kvt == "f16" else p)


@pytest.mark.parametrize("nq", [0, 9, -1])
def test_decode_rejects_bad_query_count(nq):
    with pytest.raises(ops.QwaError, match="queries"):
        ops.attn_decode_multi(0x1000, 0x1000, _kv("q8_0"), "q8_0", 10, nq, 0x1000, 0x1000)


def test_decode_rejects_context_beyond_limits():
    with pytest.raises(ops.QwaError, match="262144"):
        ops.attn_decode_multi(0x1000, 0x1000, _kv("q4_0", 300000), "q4_0", 262144, 1, 0x1000, 0x1000)
    with pytest.raises(ops.QwaError, match="capacity"):
        ops.attn_decode_multi(0x1000, 0x1000, _kv("q4_0", 100), "q4_0", 99, 2, 0x1000, 0x1000)


def test_rejects_bad_kv():
    with pytest.raises(ops.QwaError, match="unknown KV type"):
        ops.attn_decode_multi(0x1000, 0x1000, _kv("q8_0"), 5, 10, 1, 0x1000, 0x1000)
    kv = _kv("q8_0")
    kv.ks = None
    with pytest.raises(ops.QwaError, match="scale"):
        ops.attn_prefill(0x1000, 0x1000, kv, "q8_0", 4, 0, 0x1000)
    with pytest.raises(ops.QwaError, match="capacity"):
        ops.attn_prefill(0x1000, 0x1000, _kv("f16", 100), "f16", 64, 40, 0x1000)
    with pytest.raises(ops.QwaError, match="B = 0"):
        ops.attn_prefill(0x1000, 0x1000, _kv("f16", 100), "f16", 0, 0, 0x1000)


def test_kv_lifecycle_sizes_and_validation():
    # packed bytes: 4 heads x n positions x (K + V) x (values + scales)
    assert ops.kv_packed_bytes("f16", 10) == 4 * 10 * 2 * 512
    assert ops.kv_packed_bytes("q8_0", 10) == 4 * 10 * 2 * (256 + 16)
    assert ops.kv_packed_bytes("q4_0", 150000) == 150000 * 1152
    with pytest.raises(ops.QwaError, match="do not fit"):
        ops.kv_pack(_kv("q4_0", 100), "q4_0", 101, 0x1000)
    with pytest.raises(ops.QwaError, match="null packed buffer"):
        ops.kv_unpack(0, _kv("q8_0", 100), "q8_0", 10)
    ops.kv_pack(_kv("q8_0", 100), "q8_0", 0, 0x1000)  # nothing to move: returns before any copy


def test_prep_rejects_bad_row_sources():
    kv = _kv("q4_0")
    src = ops.RowSrc(0x1000, 12288)
    bad = ops.RowSrc(0x1000, 100)  # tail without host memory
    with pytest.raises(ops.QwaError, match="host tail"):
        ops.attn_prep_multi(src, bad, src, 0x1000, 0x1000, 0, 0, 1, 1e7, 1e-6, "q4_0", kv, 0x1000, 0x1000)
    with pytest.raises(ops.QwaError, match="capacity"):
        ops.attn_prep_multi(src, ops.RowSrc(0x1000, 1024), ops.RowSrc(0x1000, 1024), 0x1000, 0x1000, 1020, 0, 8,
                            1e7, 1e-6, "q4_0", kv, 0x1000, 0x1000)


def test_cpp_shim_compiles_and_links():
    """A translation unit written against the reference's q38rt::cuda names builds against the shim + library."""
    src = r'''
#include "q38rt_attn.hpp"
using namespace q38rt::cuda;
int main() {
    KVLayer kv; kv.capacity = 16;
    if (kv_value_bytes(KVType::Q4_0) != 128 || kv_scale_bytes(KVType::F16) != 0) return 1;
    if (attn_max_positions() != 262144 || attn_work_bytes(4096) == 0) return 2;
    void (*fp)(const float*, const float*, const KVLayer&, KVType, int, int, void*, float*, const ActQ8*,
               hipStream_t, float*) = attn_decode_multi;
    void (*pp)(const float*, const float*, const KVLayer&, KVType, int, int, uint16_t*, hipStream_t) = attn_prefill;
    void (*ph)(const float*, const float*, const KVLayer&, KVType, int, int, __half*, hipStream_t) = attn_prefill;
    void (*ds)(const DeltaNetParams&, const float*, const float*, const float*, const float*, int, float, float*,
               const ActQ8*, hipStream_t) = deltanet_step;
    void (*dm)(const DeltaNetParams&, int, const DNTokens&, int, int, int, float, float*, const ActQ8*,
               hipStream_t) = deltanet_multi;
    void (*dr)(const DeltaNetParams&, const float*, const float*, const float*, const float*, int, int, float, void*,
               float*, __half*, hipStream_t) = deltanet_rows;
    enum class QuantFormat : uint32_t { Q4_K = 12, IQ1_S = 19, IQ3_S = 21 };
    if (!gemv_q8_supported(QuantFormat::Q4_K) || !gemv_q8_supported(QuantFormat::IQ3_S) ||
        gemv_q8_supported(QuantFormat::IQ1_S)) return 5;
    bool (*gq)(QuantFormat, const void*, size_t, int, int, const ActQ8&, float*, hipStream_t, bool) = gemv_q8;
    bool (*gn)(QuantFormat, const void*, size_t, int, int, const ActQ8&, int, int, float*, int, hipStream_t, bool) =
        gemv_q8n;
    bool (*dq)(QuantFormat, const void*, size_t, int, int, __half*, hipStream_t) = dequant_rows_f16;
    void (*qa)(const float*, int, int, ActQ8, hipStream_t) = quantize_act_q8;
    void (*gb)(const uint16_t*, int, int, const float*, float*, hipStream_t) = gemv_bf16;
    if (!gq || !gn || !dq || !qa || !gb) return 6;
    void (*gm)(void*, const __half*, int, int, const __half*, int, int, float*, int, bool, hipStream_t) = gemm_f16;
    void* (*cc)() = cublas_create;
    bool (*cb)(void*, hipStream_t, void*, size_t) = cublas_bind;
    if (!gm || !cc || !cb) return 7;
    DNTokens tk;
    if (dn_work_bytes(1024) != ((size_t)1024 * (10240 + 2 * 2048 + 2 * 48) + 64 * 48 * 704) * 4 || tk.qkv_split != (1 << 30)) return 4;
    return (fp && pp && ph && ds && dm && dr) ? 0 : 3;
}
'''
    tmp = os.path.join(ROOT, "_build_test_shim")
    os.makedirs(tmp, exist_ok=True)
    cpp = os.path.join(tmp, "shim.cpp")
    exe = os.path.join(tmp, "shim")
    open(cpp, "w").write(src)
    libdir = os.path.dirname(ops.library_path())
    cmd = ["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"), "-I",
           "/opt/rocm/include", cpp, "-o", exe, "-L", libdir, "-lqwattn", f"-Wl,-rpath,{libdir}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, (r.returncode, r.stderr[-2000:])


def _dnp():
    return ops.DNParams(0x1000, 0x1000, 0x1000, 0x1000, 0x1000, 0x1000)


def test_deltanet_rejects_bad_arguments():
    """The reference aborts on more than DN_MAXN new tokens (src/cuda/ops.cu:959); the C ABI returns a status."""
    p = _dnp()
    tok = ops.DNTokens(qkv=0x1000, z=0x1000, beta=0x1000, alpha=0x1000)
    with pytest.raises(ops.QwaError, match="new tokens > 7"):
        ops.deltanet_multi(p, 0, tok, 0, 8, 8, 1e-6, 0x1000)
    with pytest.raises(ops.QwaError, match="conv buffer"):
        ops.deltanet_multi(p, 2, tok, 0, 1, 1, 1e-6, 0x1000)
    with pytest.raises(ops.QwaError, match="write_after"):
        ops.deltanet_multi(p, 0, tok, 0, 2, 3, 1e-6, 0x1000)
    with pytest.raises(ops.QwaError, match="saved inputs"):
        ops.deltanet_multi(p, 0, tok, 1, 1, 2, 1e-6, 0x1000)
    with pytest.raises(ops.QwaError, match="host part"):
        ops.deltanet_multi(p, 0, ops.DNTokens(qkv=0x1000, z=0x1000, beta=0x1000, alpha=0x1000, qkv_split=100), 0, 1,
                           1, 1e-6, 0x1000)
    with pytest.raises(ops.QwaError, match="incomplete DeltaNet parameters"):
        ops.deltanet_step(ops.DNParams(0x1000, 0x1000, 0x1000, 0x1000, 0x1000, None), 0x1000, 0x1000, 0x1000,
                          0x1000, 0, 1e-6, 0x1000)
    with pytest.raises(ops.QwaError, match="B = 0"):
        ops.deltanet_rows(p, 0x1000, 0x1000, 0x1000, 0x1000, 0, 0, 1e-6, 0x1000, 0x1000, 0x1000)
    # nothing to apply is not an error (the reference returns)
    ops.deltanet_multi(p, 0, ops.DNTokens(), 0, 0, 0, 1e-6, None)
