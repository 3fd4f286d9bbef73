#!/usr/bin/env python3
"""Benchmark of the gated-attention hot path on one MI355X -- prints ONE JSON line.

Headline (BASELINE.json metric): decode attention over a 150000-position Q4_0 KV cache, 24 query / 4 KV heads,
head_dim 256, one query per call.  One "step" = one token's decode attention over all 16 attention layers of the
model, each layer with its own cache (16 x 172.8 MB, so consecutive calls cannot be served from the 256 MB
Infinity Cache).  value = algorithmic HBM bytes (150000 x 1152 B per layer) / time per layer, in GB/s.
Secondary figures in the same line: 7-query verify at 150000 and 32768 positions, F16 decode at 4096 (C1), Q8_0
decode with append at 4096, and the 1024-token prefill chunk at p0 = 32768 (TFLOP/s against the fp16 MFMA dense
peak).

The CPU baseline (rank 0, N = 1 only) is the oracle's restatement of the reference CPU attention
(src/reference/ref_model.cpp:138-163: fp32 8-lane FMA dots, double softmax, OpenMP over (token, head)) on bounded
samples of the configured shapes, timed on this box's host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s
METRIC = "decode attn µs/layer + HBM GB/s @150K Q4_0 KV; prefill attn TFLOP/s (1024-tok chunk)"
# HBM bytes per k_dec4 launch at the headline workload come from the committed rocprofv3 PMC summary below.  It records
# the digest of the decode kernel's sources it was measured on; a run on other sources reports traffic null.
TRAFFIC_PROFILE = os.path.join("profiles", "decode_q4_0_150k_hbm_traffic.md")
DECODE_SOURCES = ("attn_decode.hip", "attn_decode_ilp.hip", "kv_operands.hpp", "launch.hpp", "qwattn_common.hpp")
BYTES_PER_POS = {0: 4096, 1: 2176, 2: 1152}  # K + V values and scales over the 4 KV heads
PROF_LAUNCHES = 1024  # launches one qwa_profile window times


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--positions", type=int, default=150000)
    ap.add_argument("--nq", type=int, default=1,
                    help="queries per headline call (7: the speculative-verify variant of the same workload)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="headline decode only")
    ap.add_argument("--consumer-only", action="store_true",
                    help="print only the output-projection consumer figures (GEMV, fp16 GEMM)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="print only the prefill figures (C4 and the reference's 512-token points; for profiling)")
    ap.add_argument("--deltanet-only", action="store_true",
                    help="print only the Gated DeltaNet figures (for profiling those kernels)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run 5 device copies of 512 MiB (a known-size kernel to calibrate HBM counters)")
    return ap.parse_args()


def decode_source_digest():
    """sha256 (first 16 hex digits) over the decode kernel's source files, in DECODE_SOURCES order."""
    import hashlib
    h = hashlib.sha256()
    for f in DECODE_SOURCES:
        with open(os.path.join(HERE, "qwengine_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def measured_traffic():
    """(bytes per k_dec4 launch, note) from TRAFFIC_PROFILE's machine-readable line
    `traffic: kernel=<name> source_digest=<hex> read_bytes=<R> write_bytes=<W>`; (None, why) when the summary is
    missing or was measured on other decode sources than this tree's."""
    import re
    try:
        with open(os.path.join(HERE, TRAFFIC_PROFILE)) as fh:
            text = fh.read()
    except OSError:
        return None, f"{TRAFFIC_PROFILE} missing"
    m = re.search(r"traffic: kernel=(\S+) source_digest=([0-9a-f]+) read_bytes=(\d+) write_bytes=(\d+)", text)
    if not m:
        return None, f"{TRAFFIC_PROFILE} has no traffic line"
    if m.group(2) != decode_source_digest():
        return None, f"{TRAFFIC_PROFILE} was measured on decode sources {m.group(2)}, this tree is " \
                     f"{decode_source_digest()}: re-run its PMC commands"
    return int(m.group(3)) + int(m.group(4)), f"{TRAFFIC_PROFILE} ({m.group(1)}, sources {m.group(2)})"


def fill_cache(ops, torch, kvt, n, seed, outlier_frac=0.01):
    kv = ops.KVLayer.allocate(kvt, n, zero=False)
    g = torch.Generator(device="cuda").manual_seed(seed)
    chunk = 32768
    for p in range(0, n, chunk):
        m = min(chunk, n - p)
        K = torch.randn((m, 4, 256), generator=g, device="cuda")
        V = torch.randn((m, 4, 256), generator=g, device="cuda")
        if outlier_frac:
            K[torch.rand((m, 4), generator=g, device="cuda") < outlier_frac] *= 8.0
        ops.kv_append(K, V, p, m, kvt, kv)
    return kv


SETTLE_S = 0.3  # seconds of untimed steps before a headline measurement


def settle(torch, fn, seconds=SETTLE_S):
    """Run fn untimed until `seconds` of wall time have passed (synchronising every few calls), so that the GPU's
    clocks have left their transient after idle before anything is timed."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()


def time_calls(torch, fn, reps, warmup, settle_s=SETTLE_S):
    # every workload settles first, as the headline does: a new workload after another (or after idle) starts in the
    # clock transient, which a few warmup calls do not cover
    settle(torch, fn, settle_s)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps  # ms


def time_graph(torch, fn, reps, warmup=3):
    """fn captured once into a HIP graph (as the engine runs its decode step), then timed over graph replays: the
    figure is the GPU's, not the Python launch loop's."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    ms = time_calls(torch, g.replay, reps, warmup)
    del g
    return ms


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the path has no multi-GPU "
              "collective -- run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    import qwengine_amd.ops as ops

    ops.lib()
    torch.manual_seed(0)
    if args.deltanet_only:
        print(json.dumps({"deltanet": deltanet_extras(ops, torch, args.steps)}), flush=True)
        return
    if args.consumer_only:
        print(json.dumps({"consumer": consumer_extras(ops, torch, args.steps)}), flush=True)
        return
    if args.prefill_only:
        print(json.dumps({"prefill": prefill_extras(ops, torch)}), flush=True)
        return
    n, L = args.positions, args.layers
    kvt = ops.Q4_0
    print(f"[bench] filling {L} layer caches of {n} Q4_0 positions", file=sys.stderr, flush=True)
    layers = [fill_cache(ops, torch, kvt, n, 1000 + i) for i in range(L)]
    g = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn((8, 24, 256), generator=g, device="cuda")
    gate = torch.randn((8, 24, 256), generator=g, device="cuda")
    work = torch.empty(ops.attn_work_bytes(n) // 4 + 1, dtype=torch.float32, device="cuda")
    out = torch.empty((8, 24, 256), device="cuda")

    def step(nq=args.nq):
        for kv in layers:
            ops.attn_decode_multi(q, gate, kv, kvt, n - nq, nq, work, out)

    # ---- headline: the GPU's clock settling, W warmup steps, then exactly K timed steps.  After the caches are filled
    # the per-step time of this workload rises from ~40 to ~53 us per layer within a few steps and settles at ~39 us
    # only after ~25-30 steps (~18 ms of decode work, the GPU's power management adjusting its clocks; again after 2 s
    # idle), so a few warmup steps would time the transient.  Untimed steps for SETTLE_S seconds come first, so that
    # the K timed steps measure the steady state an engine decoding continuously runs at.
    settle(torch, step)
    print(f"[bench] decode: {args.warmup} warmup + {args.steps} timed steps", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    # the dominant kernel alone: HIP events holding each split-K decode launch's own start / end timestamps (same
    # stream, hipExtLaunchKernelGGL inside the library's timing window), over the same work
    # (the window holds PROF_LAUNCHES launches: at most that many calls are timed, one split-K launch per call)
    prof_steps = max(1, min(args.steps, PROF_LAUNCHES // L))
    ops.profile_begin()
    for _ in range(prof_steps):
        step()
    kern_ms, kern_n = ops.profile_end()
    calls = prof_steps * L
    kern_us = kern_ms * 1000.0 / calls
    kern_dev_us = ops.profile_device_ms() * 1000.0 / calls
    kern_mhz = ops.profile_clock_mhz()
    us_layer = ms_per_step * 1000.0 / L
    if args.copy_probe:
        src = torch.empty(1 << 27, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    bytes_layer = n * BYTES_PER_POS[kvt]
    traffic, traffic_note = measured_traffic() if (n, args.nq) == (150000, 1) else \
        (None, "PMC traffic is measured for the headline workload only")
    gbs = bytes_layer / (us_layer * 1e-6) / 1e9

    result = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (K/V ~N(0,1), 1% of key rows x8, quantized on append; random gate logits)",
        "config": {"workload": ("decode" if args.nq == 1 else f"verify{args.nq}") + f"_q4_0_{n // 1000}k", "kv": "q4_0",
                   "positions": n, "queries_per_call": args.nq,
                   "layers_per_step": L, "q_heads": 24, "kv_heads": 4, "head_dim": 256},
        "decode_us_per_layer": round(us_layer, 3),
        "roofline": {"bound": "hbm", "achieved": round(bytes_layer / (kern_us * 1e-6) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(bytes_layer / (kern_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "traffic_source": traffic_note,
                     "kernel": "k_dec4 (split-K Q4_0 decode), kernel time per call averaged over the timed calls",
                     "kernel_us": round(kern_us, 3), "launches": kern_n, "calls": calls,
                     "kernel_us_device_clock": round(kern_dev_us, 3),
                     "kernel_clock_mhz": round(kern_mhz, 1),
                     "algorithmic_bytes_per_launch": bytes_layer},
    }

    if not args.no_extra:
        extra = {}
        # 7-query speculative verify over the same 150000-position caches
        ms = time_calls(torch, lambda: step(7), max(5, args.steps // 5), 2)
        us = ms * 1000.0 / L
        extra["verify7_150k_us_per_layer"] = round(us, 3)
        extra["verify7_150k_gbs"] = round((n + 6) * BYTES_PER_POS[kvt] / (us * 1e-6) / 1e9, 1)
        # the same 16 layers captured in one HIP graph, as an engine issues its step (no Python launch gaps)
        ms = time_graph(torch, lambda: step(7), max(5, args.steps // 5))
        extra["verify7_150k_us_per_layer_graph"] = round(ms * 1000.0 / L, 3)
        del layers
        torch.cuda.empty_cache()
        # C3: 7-query verify over Q4_0 32768 (16 layers)
        n3 = 32768 + 7
        l3 = [fill_cache(ops, torch, ops.Q4_0, n3, 2000 + i) for i in range(L)]
        ms = time_calls(torch, lambda: [ops.attn_decode_multi(q, gate, kv, ops.Q4_0, 32768, 7, work, out) for kv in l3],
                        max(5, args.steps // 5), 2)
        us = ms * 1000.0 / L
        extra["verify7_q4_32768_us_per_layer"] = round(us, 3)
        extra["verify7_q4_32768_gbs"] = round(n3 * 1152 / (us * 1e-6) / 1e9, 1)
        ms = time_graph(torch, lambda: [ops.attn_decode_multi(q, gate, kv, ops.Q4_0, 32768, 7, work, out) for kv in l3],
                        max(5, args.steps // 5))
        extra["verify7_q4_32768_us_per_layer_graph"] = round(ms * 1000.0 / L, 3)
        del l3
        # the other two cache formats at the headline context: decode and 7-query verify over 150000 positions
        # (4 layers each, rotated; 1.3 GB (Q8_0) and 2.5 GB (F16) per rotation, past the MALL)
        for kvo, nm in ((ops.Q8_0, "q8_0"), (ops.F16, "f16")):
            lo = [fill_cache(ops, torch, kvo, n + 8, 4000 + 10 * kvo + i) for i in range(4)]
            for nqo in (1, 7):
                ms = time_graph(torch, lambda: [ops.attn_decode_multi(q, gate, kv, kvo, n + 7 - nqo, nqo, work, out)
                                                for kv in lo], max(5, args.steps // 5))
                us = ms * 1000.0 / len(lo)
                extra[f"{'decode' if nqo == 1 else 'verify7'}_{nm}_150k_us_per_layer_graph"] = round(us, 3)
                extra[f"{'decode' if nqo == 1 else 'verify7'}_{nm}_150k_gbs"] = round(
                    (n + 7) * BYTES_PER_POS[kvo] / (us * 1e-6) / 1e9, 1)
            del lo
            torch.cuda.empty_cache()
        # C1: F16 4096 decode, one query (the CPU-runnable case; 16 layers of 16.8 MB)
        l1 = [fill_cache(ops, torch, ops.F16, 4097, 5000 + i, 0.0) for i in range(L)]
        ms = time_calls(torch, lambda: [ops.attn_decode_multi(q, gate, kv, ops.F16, 4096, 1, work, out) for kv in l1],
                        max(5, args.steps // 5), 2)
        extra["decode_f16_4096_us_per_layer"] = round(ms * 1000.0 / L, 3)
        ms = time_graph(torch, lambda: [ops.attn_decode_multi(q, gate, kv, ops.F16, 4096, 1, work, out) for kv in l1],
                        max(5, args.steps // 5))
        extra["decode_f16_4096_us_per_layer_graph"] = round(ms * 1000.0 / L, 3)
        extra["decode_f16_4096_gbs_graph"] = round(4097 * 4096 / (ms * 1e-3 / L) / 1e9, 1)
        del l1
        # C2: Q8_0 4096 decode with the new token's quantize-on-append (append + decode per layer)
        l2 = [fill_cache(ops, torch, ops.Q8_0, 4097, 3000 + i, 0.0) for i in range(L)]
        knew = torch.randn((1, 4, 256), device="cuda")
        vnew = torch.randn((1, 4, 256), device="cuda")

        def c2():
            for kv in l2:
                ops.kv_append(knew, vnew, 4096, 1, ops.Q8_0, kv)
                ops.attn_decode_multi(q, gate, kv, ops.Q8_0, 4096, 1, work, out)
        ms = time_calls(torch, c2, max(5, args.steps // 5), 2)
        extra["decode_q8_4096_append_us_per_layer"] = round(ms * 1000.0 / L, 3)
        ms = time_graph(torch, c2, max(5, args.steps // 5))
        extra["decode_q8_4096_append_us_per_layer_graph"] = round(ms * 1000.0 / L, 3)
        del l2
        extra.update(prefill_extras(ops, torch))
        extra.update(deltanet_extras(ops, torch, args.steps))
        extra.update(consumer_extras(ops, torch, args.steps))
        result["extra"] = extra

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(ops, torch, n)
    print(json.dumps(result), flush=True)


def prefill_extras(ops, torch):
    """The 1024-token prefill chunk at p0 = 32768 over Q8_0 (C4; TFLOP/s against the fp16 MFMA dense peak, whole call
    and the MFMA kernel alone) and the reference's own 512-token bench points."""
    out = {}
    # C4: prefill chunk of 1024 tokens at p0 = 32768, Q8_0
    p0, B = 32768, 1024
    kv4 = fill_cache(ops, torch, ops.Q8_0, p0 + B, 4000, 0.0)
    qp = torch.randn((B, 24, 256), device="cuda").half().float()
    gp = torch.randn((B, 24, 256), device="cuda")
    o16 = torch.empty((B, 24, 256), dtype=torch.float16, device="cuda")
    ops.attn_prefill_reserve(B, p0 + B)  # set-up: the stream's prefill workspace
    # clocks settled (see the headline), then the median of 4 groups of 5 calls
    settle(torch, lambda: ops.attn_prefill(qp, gp, kv4, ops.Q8_0, B, p0, o16))
    ms = sorted(time_calls(torch, lambda: ops.attn_prefill(qp, gp, kv4, ops.Q8_0, B, p0, o16), 5, 0, settle_s=0.0)
                for _ in range(4))[1:3]
    ms = sum(ms) / 2
    ops.profile_begin()
    for _ in range(10):
        ops.attn_prefill(qp, gp, kv4, ops.Q8_0, B, p0, o16)
    pk_ms, pk_n = ops.profile_end()
    out["prefill_kernel_ms"] = round(pk_ms / max(pk_n, 1), 4)
    out["prefill_kernel_ms_device_clock"] = round(ops.profile_device_ms() / max(pk_n, 1), 4)
    # the shader clock the kernel ran at, and its MFMA rate against the dense fp16 peak at that clock (256 CUs x 4
    # SIMDs x 1024 fp16 flop per clock; 2.52 PFLOP/s at the 2.4 GHz that the published peak assumes)
    mhz = ops.profile_clock_mhz()
    out["prefill_kernel_clock_mhz"] = round(mhz, 1)
    flop = 4.0 * 24 * 256 * sum(p0 + t + 1 for t in range(B))
    tflops = flop / (ms * 1e-3) / 1e12
    out["prefill_1024_at_32768_ms"] = round(ms, 4)
    out["prefill_tflops"] = round(tflops, 1)
    out["prefill_mfma_frac"] = round(tflops / MFMA_F16_PEAK_TFLOPS, 4)
    out["prefill_kernel_mfma_frac"] = round(flop / (out["prefill_kernel_ms"] * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)
    if mhz > 0:
        out["prefill_kernel_mfma_frac_at_clock"] = round(
            flop / (out["prefill_kernel_ms"] * 1e-3) / (256 * 4 * 1024 * mhz * 1e6), 4)
    del kv4
    # the reference's own prefill bench points (tests/kernels/test_attn_prefill.cu:79-101): B = 512 chunks at
    # p0 = 7680, 32256, 99488 over Q8_0, flop = 4 B 24 256 (p0 + B / 2) as it counts them
    B = 512
    kvr = fill_cache(ops, torch, ops.Q8_0, 99488 + B, 4100, 0.0)
    ops.attn_prefill_reserve(B, 99488 + B)
    for p0 in (7680, 32256, 99488):
        settle(torch, lambda: ops.attn_prefill(qp[:B], gp[:B], kvr, ops.Q8_0, B, p0, o16[:B]))
        ms = sorted(time_calls(torch, lambda: ops.attn_prefill(qp[:B], gp[:B], kvr, ops.Q8_0, B, p0, o16[:B]),
                               5, 0, settle_s=0.0) for _ in range(4))[1:3]
        ms = sum(ms) / 2
        out[f"prefill_512_at_{p0}_ms"] = round(ms, 4)
        out[f"prefill_512_at_{p0}_tflops"] = round(4.0 * B * 24 * 256 * (p0 + B / 2) / (ms * 1e-3) / 1e12, 1)
    del kvr
    return out


def deltanet_extras(ops, torch, steps, L=48):
    """Gated DeltaNet layers (48 of them as in the model, each with its own 3.1 MB state): one decode token per layer,
    a 7-token verify with the lazy commit of the first token (both as HIP-graph replays of the 36 layers, which is how the
    engine issues its decode step), and a 1024-token prefill chunk.  Algorithmic HBM bytes per decode
    layer: the state read and written (2 x 48 x 128 x 128 x 4) plus the conv window, conv weights and the token's rows."""
    ch, vd, vh = ops.DN_CH, ops.DN_VD, ops.DN_VH
    g = torch.Generator(device="cuda").manual_seed(5)
    rn = lambda *s, sc=1.0: torch.randn(*s, device="cuda", generator=g) * sc
    layers = [ops.DNParams(rn(ch, 4, sc=0.5), rn(vh), -torch.exp(rn(vh, sc=0.5)), 1.0 + rn(128, sc=0.1),
                           rn(2, 3, ch, sc=0.5), rn(vh, 128, 128, sc=0.1)) for _ in range(L)]
    qkv, z = rn(7, ch, sc=0.5), rn(7, vd)
    b, a = rn(7, 64), rn(7, 64, sc=2.0)
    o = torch.empty((7, vd), device="cuda")
    tk1 = ops.DNTokens(qkv=qkv, z=z, beta=b, alpha=a)

    def dec():
        for p in layers:
            ops.deltanet_multi(p, 0, tk1, 0, 1, 1, 1e-6, o)
    out = {}
    ms = time_graph(torch, dec, max(10, steps))
    us = ms * 1000.0 / L
    state_bytes = 2 * vh * 128 * 128 * 4
    dec_bytes = state_bytes + 6 * ch * 4 + ch * 16 + (ch + 2 * vd) * 4  # + conv window r/w, conv_w, rows
    out["deltanet_decode_us_per_layer"] = round(us, 3)
    out["deltanet_decode_gbs"] = round(dec_bytes / (us * 1e-6) / 1e9, 1)
    sq, sb, sa = torch.empty_like(qkv), torch.empty_like(b), torch.empty_like(a)
    tk7 = ops.DNTokens(qkv=qkv, z=z, beta=b, alpha=a, oqkv=sq, obeta=sb, oalpha=sa)

    def ver():
        for p in layers:
            ops.deltanet_multi(p, 0, tk7, 0, 7, 1, 1e-6, o)
    ms = time_graph(torch, ver, max(5, steps // 2))
    out["deltanet_verify7_us_per_layer"] = round(ms * 1000.0 / L, 3)
    B = 1024
    xq, xz = rn(B, ch, sc=0.5), rn(B, vd)
    xb, xa = rn(B, vh), rn(B, vh, sc=2.0)
    work = torch.empty(ops.dn_work_bytes(B) // 4, device="cuda")
    core = torch.empty((B, vd), device="cuda")
    o16 = torch.empty((B, vd), dtype=torch.float16, device="cuda")
    p0 = layers[0]
    ms = time_calls(torch, lambda: ops.deltanet_rows(p0, xq, xz, xb, xa, B, 0, 1e-6, work, core, o16), 10, 2)
    out["deltanet_prefill_1024_ms"] = round(ms, 4)
    out["deltanet_prefill_tokens_per_s"] = round(B / (ms * 1e-3), 0)
    del layers
    torch.cuda.empty_cache()
    return out


def consumer_extras(ops, torch, steps):
    """The attention output's consumers at the O-projection shape (6144 inputs, 5120 outputs): the decode GEMV over
    one ActQ8 column (weights streamed once: bytes = the weight matrix) for two formats, as HIP-graph replays of 16
    calls, and the prefill FP16 GEMM of a 1024-token chunk on hipBLASLt."""
    import numpy as np
    sys.path.insert(0, os.path.join(HERE, "tests"))
    K, N = 6144, 5120
    out = {}
    x = torch.randn((1, K), device="cuda")
    a = ops.ActQ8.allocate(K)
    ops.quantize_act_q8(x, K, 1, a)
    y = torch.empty(N, device="cuda")
    rng = np.random.default_rng(0)
    for fmt, name in ((ops.W_Q4_K, "q4_k"), (ops.W_IQ4_XS, "iq4_xs"), (ops.W_IQ3_S, "iq3_s"), (ops.W_IQ2_XS, "iq2_xs"),
                      (ops.W_IQ2_XXS, "iq2_xxs"), (ops.W_IQ2_S, "iq2_s")):
        rb = ops.w_row_bytes(fmt, K)
        Wn = rng.integers(0, 256, (N, rb), dtype=np.uint8)
        blocks = Wn.reshape(N, K // 256, rb // (K // 256))
        blocks[:, :, 1] = 0x1c  # every d (and Q4_K's dmin) field a small fp16 value: bytes xx 1c ~ 0.004
        if fmt == ops.W_Q4_K:
            blocks[:, :, 3] = 0x1c
        # enough copies to pass 300 MB, so that neither the L2s nor the 256 MB MALL serve the weights
        nw = -(-300_000_000 // (N * rb))
        W = [torch.from_numpy(Wn).cuda() for _ in range(nw)]

        def run():
            for i in range(16):
                ops.gemv_q8(fmt, W[i % nw], rb, K, N, a, y)
        ms = time_graph(torch, run, max(5, steps // 5))
        us = ms * 1000.0 / 16
        out[f"gemv_{name}_6144x5120_us"] = round(us, 3)
        out[f"gemv_{name}_6144x5120_gbs"] = round(N * rb / (us * 1e-6) / 1e9, 1)
        del W
    B = 1024
    g = ops.Gemm()
    Wh = (torch.randn((N, K), device="cuda") * 0.05).half()
    Xh = torch.randn((B, K), device="cuda").half()
    Y = torch.empty((B, N), device="cuda")
    ms = time_calls(torch, lambda: g.f16(Wh, N, K, Xh, K, B, Y, N), max(10, steps // 2), 3)
    out["gemm_f16_1024x5120x6144_ms"] = round(ms, 4)
    out["gemm_f16_tflops"] = round(2.0 * B * N * K / (ms * 1e-3) / 1e12, 1)
    # the same shape after qwa_gemm_tune (set-up time measurement of hipBLASLt's candidates)
    g.tune(Wh, N, K, Xh, K, B, Y, N, max_candidates=32)
    ms = time_calls(torch, lambda: g.f16(Wh, N, K, Xh, K, B, Y, N), max(10, steps // 2), 3)
    out["gemm_f16_tuned_1024x5120x6144_ms"] = round(ms, 4)
    out["gemm_f16_tuned_tflops"] = round(2.0 * B * N * K / (ms * 1e-3) / 1e12, 1)
    g.close()
    return out


def cpu_baseline(ops, torch, n):
    """The reference CPU arithmetic (oracle mode 1: src/reference/ref_model.cpp:138-163, fp32 8-lane FMA dots, double
    softmax and P.V, OpenMP over (token, head)) on this box's host threads, at the four shapes of the CPU plan: C1
    (F16 4096, one query; the tensors of the C1 GPU parity test), C3 (7 queries over Q4_0 32768) and the headline
    shape (Q4_0 150000) with 1 and 7 queries.  Quantized caches are dequantized to fp32 first, as the reference CPU
    path holds fp32 K / V.  Each shape runs for about 3 s after one warm-up call."""
    import numpy as np
    import oracle as O
    sys.path.insert(0, os.path.join(HERE, "tests"))
    from kvutil import c1_inputs
    print("[bench] cpu baseline", file=sys.stderr, flush=True)
    threads = O.max_threads()
    rng = np.random.default_rng(7)
    qn = rng.standard_normal((8, 24, 256)).astype(np.float32)
    gn = rng.standard_normal((8, 24, 256)).astype(np.float32)

    def host_cache(kvt, kv):
        K = O.kv_load_rows(kvt, kv.k.cpu().numpy(), kv.ks.cpu().numpy().view(np.uint16) if kv.ks is not None else
                           np.zeros((4, kv.capacity, 8), np.uint16))
        V = O.kv_load_rows(kvt, kv.v.cpu().numpy(), kv.vs.cpu().numpy().view(np.uint16) if kv.vs is not None else
                           np.zeros((4, kv.capacity, 8), np.uint16))
        return K, V

    def timed(q, g, K, V, pos0, nq, budget=3.0):
        O.attention(q, g, K, V, pos0, nq, mode=1)  # warm-up
        reps, t0 = 0, time.perf_counter()
        while reps < 2 or time.perf_counter() - t0 < budget:
            O.attention(q, g, K, V, pos0, nq, mode=1)
            reps += 1
        return (time.perf_counter() - t0) / reps, reps

    shapes = {}
    kv1, q1, g1 = c1_inputs()
    K, V = host_cache(ops.F16, kv1)
    dt, reps = timed(q1.cpu().numpy(), g1.cpu().numpy(), K, V, 4095, 1)
    shapes["c1_f16_4096_nq1"] = {"us_per_layer": round(dt * 1e6, 1), "gbs": round(4096 * 4096 / dt / 1e9, 3),
                                 "reps": reps}
    del kv1, K, V
    kv3 = fill_cache(ops, torch, ops.Q4_0, 32768 + 7, 2000)
    K, V = host_cache(ops.Q4_0, kv3)
    dt, reps = timed(qn[:7], gn[:7], K, V, 32768, 7)
    shapes["c3_q4_0_32768_nq7"] = {"us_per_layer": round(dt * 1e6, 1), "gbs": round(32775 * 1152 / dt / 1e9, 3),
                                   "reps": reps}
    del kv3, K, V
    kv = fill_cache(ops, torch, ops.Q4_0, n, 1000)
    K, V = host_cache(ops.Q4_0, kv)
    del kv
    dt1, reps1 = timed(qn[:1], gn[:1], K, V, n - 1, 1)
    shapes["c5_q4_0_150k_nq1"] = {"us_per_layer": round(dt1 * 1e6, 1), "gbs": round(n * 1152 / dt1 / 1e9, 3),
                                  "reps": reps1}
    dt, reps = timed(qn[:7], gn[:7], K, V, n - 7, 7)
    shapes["c5_q4_0_150k_nq7"] = {"us_per_layer": round(dt * 1e6, 1), "gbs": round(n * 1152 / dt / 1e9, 3),
                                  "reps": reps}
    return {"value": shapes["c5_q4_0_150k_nq1"]["gbs"], "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_layer": shapes["c5_q4_0_150k_nq1"]["us_per_layer"], "shapes": shapes,
            "sample": f"decode calls of the reference CPU arithmetic (oracle mode 1, {threads} OpenMP threads) over "
                      "fp32 caches: C1 F16 4096 nq=1, C3 Q4_0 32768 nq=7, Q4_0 150000 nq=1 (value) and nq=7; about "
                      "3 s per shape"}


if __name__ == "__main__":
    main()
