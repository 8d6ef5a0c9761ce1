"""Benchmark of the block-scaled FP8 GEMM path on one MI355X.

Workload (the config the metric's decode figure is quoted on): DeepSeek-V3
decode FP8 block-scaled GEMM, M in {1, 4, 16, 64, 128} x (N, K) in {(2112, 7168), (24576, 1536),
(7168, 16384)}. One step = for each of the 15 (M, N, K): per_group_quant_fp8 of the bf16 activations
(N(0,1), 1% x20 outliers) then the 128x128-block-scaled GEMM against e4m3 weights (N(0,0.02), 128x128
fp32 block scales) in aiter's preshuffled layout with the quantizer's column-major scales, bf16 out.
Each step is one HIP graph. Every GEMM of a step reads its own weight copy: a shape's five GEMMs (one
per M) take five consecutive copies of a rotation of > 512 MB per shape, so no copy is read again
before more than a step's worth of other bytes (888 MB) has passed through the 256 MB MALL -- weights
stream from HBM, as in serving.

value = whole-step algorithmic bytes / step time, in GB/s (bytes per GEMM: M*K + 4*M*K/128 + N*K +
4*ceil(N/128)*K/128 + 2*M*N; per quant: 3.03125*M*K).
roofline: the dominant kernel, the stream (decode) GEMM at M=16, (N, K) = (7168, 16384) (117.97 MB per
launch), timed alone with HIP events on its stream over graph replays; peak 8 TB/s.
roofline.traffic: HBM bytes per launch of that kernel from two rocprofv3 --pmc runs (FETCH_SIZE, then
WRITE_SIZE) of ``python3 bench.py --probe-traffic``, each scaled by what the counter reads for a plain
copy of known size in the same run; read from the committed profiles/ summary (null when absent).
decode_fused_quant: the same step with each pair made one quant_gemm_a8w8_blockwise_scaled call (one
launch at M <= 16), ms per step and its speedup over the two-op step (an extra: value keeps the
reference's two-op flow).
reference_recorded_fp8: the FP8 GEMM on the 17 shapes whose times the reference records in its kernel
schema files (its CI: graph replay after a 1 GiB cache flush, median), next to those times. Here each call
runs on cold operands too (rotating > 512 MB of copies), and the figure is the median of 7 replays after
>= 50 ms of warm-up replays. Below ~10 us the reference's figure includes its
timer's ~4.2 us floor, so only the larger shapes compare kernels.
prefill / mxfp4: extra figures (TFLOP/s vs the dense FP8 5.0 PF / MXFP4 10.1 PF peaks): FP8 at
M in {1024, 4096, 8192}, MXFP4 at M in {1, 32, 512, 4096} (M <= 32 as GB/s vs 8 TB/s). Every call reads
cold operands: a graph runs the GEMM over rotating copies of its operands (activations and weights,
> 512 MB in all), and a figure is the median over 10 replays, after >= 50 ms of warm-up replays, of the
replay time over the copies.
decode_floor: the same timing of a kernel that only reads each decode shape's M=1 bytes (the calibration
kernel aklr_probe_hbm_read, best launch shape) and of an empty kernel: the floor a decode GEMM of that
size cannot beat here.
quant: the three activation quantizers at H=7168, T in {2048, 16384} (rows a1/a4/a5), next to the
reference's recorded times where it has them.
moe: the grouped DeepSeek-V3 FP8 MoE experts (256 routed + 1 shared, top-8,
D=7168, I=2048, e4m3 weights with 128x128 scales) on Zipf(1.1) routing at T in {64, 4096}: time per
call, touched-weight bytes / time vs 8 TB/s, and TFLOP/s vs 5.0 PF.
cpu_baseline: the CPU oracle (numpy quantize, dequantize, fp32 matmul: the reference check's formula)
on one whole decode step (the same 15 quantize-then-GEMM pairs), timed on the host in the same run:
the median of 3 repetitions after a warm-up one.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
MXFP4_PEAK_TFLOPS = 10100.0


def gemm8_bytes(m, n, k):
    return m * k + 4 * m * k // 128 + n * k + 4 * (-(-n // 128)) * (k // 128) + 2 * m * n


def quant8_bytes(m, k):
    return 2 * m * k + m * k + 4 * m * k // 128


def gemm4_bytes(m, n, k):
    return (m + n) * k // 2 + (m + n) * k // 32 + 2 * m * n


def _copies(bytes_per_copy, target=512 * 2**20, lo=2):
    return max(lo, math.ceil(target / bytes_per_copy))


def _replay_time_ms(graphs, steps, warmup, stream):
    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        graphs[i % len(graphs)].replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def _replay_median_ms(graph, reps, warmup, stream, warm_ms=50.0):
    """Median over ``reps`` single replays of ``graph``, each timed with HIP events on ``stream``, after
    ``warmup`` replays and at least ``warm_ms`` of them (the clocks settle under sustained load: the first
    milliseconds of a compute-bound shape run up to 15% slower)."""
    t0 = time.perf_counter()
    n = 0
    while n < warmup or (time.perf_counter() - t0) * 1e3 < warm_ms:
        graph.replay()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        graph.replay()
        end.record(stream)
        end.synchronize()
        times.append(start.elapsed_time(end))
    times.sort()
    return times[len(times) // 2]


def _capture(fn, stream):
    fn()  # eager run first: any lazy init happens outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    return g


def build_decode(dev, shuffled=True):
    import aklr_amd
    from aklr_amd import layouts, workloads

    shapes = workloads.DEEPSEEK_NK
    ms = workloads.DECODE_M
    weights = {}
    for (n, k) in shapes:
        per = gemm8_bytes(0, n, k)
        copies = []
        for r in range(_copies(per, lo=4)):
            b, bs = workloads.blockwise_fp8_weight(n, k, seed=100 + r, device=dev)
            copies.append((layouts.shuffle_weight(b) if shuffled else b, bs))
        weights[(n, k)] = copies
    xs = {(m, k): workloads.activations(m, k, seed=m * 7 + k, device=dev) for m in ms for (_, k) in shapes}
    # step r's GEMM i of a shape reads copy (r * len(ms) + i) of that shape's rotation; enough steps to
    # go round the longest rotation
    n_sets = max(-(-len(c) // len(ms)) for c in weights.values())

    def step_fn(r):
        def run():
            for (n, k) in shapes:
                rot = weights[(n, k)]
                for i, m in enumerate(ms):
                    b, bs = rot[(r * len(ms) + i) % len(rot)]
                    q, s = aklr_amd.per_group_quant_fp8(xs[(m, k)])
                    if shuffled:
                        aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s.view(m, k // 128), bs,
                                                            operand_format="none:preshuffled")
                    else:
                        aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s, bs, scale_major_mode="MN")
        return run

    step_bytes = sum(gemm8_bytes(m, n, k) + quant8_bytes(m, k) for (n, k) in shapes for m in ms)
    return step_fn, n_sets, step_bytes, weights, xs


def fused_step_fn(weights, xs, shuffled):
    """The decode step through quant_gemm_a8w8_blockwise_scaled: the same 15 quantize-then-GEMM pairs,
    one call each (one launch at M <= 16 where the GEMM quantizes its own activations: 2112x7168 and
    24576x1536; 7168x16384's long-K plan runs the two kernels)."""
    import aklr_amd
    from aklr_amd import workloads

    fmt = "none:preshuffled" if shuffled else "none:none"

    ms = workloads.DECODE_M

    def step_fn(r):
        def run():
            for (n, k) in workloads.DEEPSEEK_NK:
                rot = weights[(n, k)]
                for i, m in enumerate(ms):
                    b, bs = rot[(r * len(ms) + i) % len(rot)]
                    aklr_amd.quant_gemm_a8w8_blockwise_scaled(xs[(m, k)], b, bs, operand_format=fmt)
        return run
    return step_fn


def time_gemm8(dev, m, n, k, weights, steps, stream, shuffled=True, calls_per_graph=None):
    """Average duration of one GEMM launch (all kernels of the op) at (m, n, k), rotating over the
    weight copies inside one graph, from HIP events on the launch stream."""
    import aklr_amd
    from aklr_amd import workloads

    x = workloads.activations(m, k, seed=5, device=dev)
    q, s = aklr_amd.per_group_quant_fp8(x)
    copies = weights[(n, k)]
    calls = calls_per_graph or len(copies)

    def run():
        for i in range(calls):
            b, bs = copies[i % len(copies)]
            if shuffled:
                aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s.view(m, k // 128), bs, operand_format="none:preshuffled")
            else:
                aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s, bs, scale_major_mode="MN")

    g = _capture(run, stream)
    ms = _replay_time_ms([g], steps, 2, stream)
    return ms / calls


def prefill_figures(dev, stream, steps=10):
    """FP8 prefill: each call on cold operands, rotating > 512 MB of (activation, weight)
    copies inside one graph; the median replay time over the copies."""
    import aklr_amd
    from aklr_amd import layouts, workloads

    out = []
    for m, (n, k) in ((m, nk) for m in workloads.PREFILL_M for nk in workloads.DEEPSEEK_NK):
        copies = []
        for r in range(_copies(gemm8_bytes(m, n, k), lo=2)):
            x = workloads.activations(m, k, seed=1 + r, device=dev)
            q, s = aklr_amd.per_group_quant_fp8(x)
            b, bs = workloads.blockwise_fp8_weight(n, k, seed=2 + r, device=dev)
            copies.append((q, s.view(m, k // 128), layouts.shuffle_weight(b), bs))
            del x, b

        def run(copies=copies):
            for q, s, b, bs in copies:
                aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s, bs, operand_format="none:preshuffled")

        g = _capture(run, stream)
        t = _replay_median_ms(g, steps, 2, stream) / len(copies)
        del g, copies
        torch.cuda.empty_cache()
        tf = 2.0 * m * n * k / (t * 1e-3) / 1e12
        out.append({"m": m, "n": n, "k": k, "us": round(t * 1e3, 2), "tflops": round(tf, 1),
                    "frac_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4)})
    return out


# The reference's recorded CI times for gemm_a8w8_blockwise_scaled (graph replay after a 1 GiB cache
# flush, median; its profiled timer has a floor of about 4.2 us a kernel): (m, n, k, variant, us, source).
_FLY = "aklr/ops/gemm/impls/flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_"
_TRI = "aklr/ops/gemm/impls/triton/gemm_a8w8_blockwise_scaled_"
REFERENCE_RECORDED = [
    (4096, 4096, 8192, "b_shuffled", 146.0, _FLY + "n4096_k8192/d9ecfacca235649e.json:201"),
    (2048, 4096, 8192, "b_shuffled", 76.5, _FLY + "n4096_k8192/d9ecfacca235649e.json:193"),
    (1024, 4096, 8192, "b_shuffled", 48.2, _FLY + "n4096_k8192/d9ecfacca235649e.json:185"),
    (4096, 32768, 1024, "b_shuffled", 152.0, _FLY + "n32768_k1024/4c06f271b8dcae0c.json:201"),
    (4096, 4096, 4096, "b_shuffled", 73.4, _FLY + "n4096_k4096/78e6bbcadf087b68.json:201"),
    (4096, 8192, 1024, "b_shuffled", 40.9, _FLY + "n8192_k1024/5af76bde5712711d.json:201"),
    (8192, 3072, 1536, "row_major", 48.1, _TRI + "n3072_k1536/4a159c69e56742a3.json:105"),
    (4096, 3072, 1536, "row_major", 25.6, _TRI + "n3072_k1536/a93ffba3bd75cf4c.json:105"),
    (2048, 3072, 1536, "row_major", 17.2, _TRI + "n3072_k1536/9cf51249fe32228f.json:105"),
    (256, 7168, 2048, "row_major", 11.2, _TRI + "n7168_k2048/fee7e092eab87fc5.json:105"),
    (128, 7168, 2048, "row_major", 8.18, _TRI + "n7168_k2048/1bbf98a368b3fcba.json:105"),
    (128, 4096, 8192, "b_shuffled", 14.3, _FLY + "n4096_k8192/d9ecfacca235649e.json:161"),
    (16, 4096, 8192, "b_shuffled", 8.38, _FLY + "n4096_k8192/d9ecfacca235649e.json:137"),
    (1, 4096, 8192, "b_shuffled", 7.79, _FLY + "n4096_k8192/d9ecfacca235649e.json:105"),
    (16, 65536, 1536, "b_shuffled", 16.6, _FLY + "n65536_k1536/95f46e6ce3030a27.json:137"),
    (1, 65536, 1536, "b_shuffled", 16.5, _FLY + "n65536_k1536/95f46e6ce3030a27.json:105"),
    (1, 32768, 1024, "b_shuffled", 7.13, _FLY + "n32768_k1024/4c06f271b8dcae0c.json:105"),
]


# Every point the reference records for gemm_a8w8_blockwise_scaled at m >= 64 (below that its times sit on
# its timer's floor), all three layout variants: (n, k, variant, schema directory under
# aklr/ops/gemm/impls/, [(m, us, file:line)]).
# bench.py --probe-reference-all runs them all; the default run times REFERENCE_RECORDED above.
REFERENCE_ALL = [
    (1024, 4096, "b_shuffled", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_n1024_k4096", [
        (64, 4.98, "2ab6fdd5f7487f88.json:153"), (128, 6.64, "2ab6fdd5f7487f88.json:161"),
        (256, 6.9, "2ab6fdd5f7487f88.json:169"), (512, 8.55, "2ab6fdd5f7487f88.json:177"),
        (1024, 11.3, "2ab6fdd5f7487f88.json:185"), (2048, 18.2, "2ab6fdd5f7487f88.json:193"),
        (4096, 30.8, "2ab6fdd5f7487f88.json:201")]),
    (1536, 4096, "b_shuffled", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_n1536_k4096", [
        (64, 5.33, "b74d90fec78ced01.json:153"), (128, 7.07, "b74d90fec78ced01.json:161"),
        (256, 9.14, "b74d90fec78ced01.json:169"), (512, 10.5, "b74d90fec78ced01.json:177"),
        (1024, 13.8, "b74d90fec78ced01.json:185"), (2048, 21.4, "b74d90fec78ced01.json:193"),
        (4096, 34.2, "b74d90fec78ced01.json:201")]),
    (32768, 1024, "b_shuffled", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_n32768_k1024", [
        (64, 9.56, "4c06f271b8dcae0c.json:153"), (128, 10.2, "4c06f271b8dcae0c.json:161"),
        (256, 16.0, "4c06f271b8dcae0c.json:169"), (512, 23.0, "4c06f271b8dcae0c.json:177"),
        (1024, 40.9, "4c06f271b8dcae0c.json:185"), (2048, 77.7, "4c06f271b8dcae0c.json:193"),
        (4096, 152.0, "4c06f271b8dcae0c.json:201")]),
    (4096, 1024, "b_shuffled", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_n4096_k1024", [
        (64, 4.92, "ad38f325b185a922.json:153"), (128, 6.48, "ad38f325b185a922.json:161"),
        (256, 7.02, "ad38f325b185a922.json:169"), (512, 8.63, "ad38f325b185a922.json:177"),
        (1024, 12.7, "ad38f325b185a922.json:185"), (2048, 17.4, "ad38f325b185a922.json:193"),
        (4096, 31.9, "ad38f325b185a922.json:201")]),
    (4096, 2048, "b_shuffled", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_n4096_k2048", [
        (64, 5.5, "5c97ff66d898f5a1.json:153"), (128, 5.93, "5c97ff66d898f5a1.json:161"),
        (256, 7.79, "5c97ff66d898f5a1.json:169"), (512, 11.4, "5c97ff66d898f5a1.json:177"),
        (1024, 15.8, "5c97ff66d898f5a1.json:185"), (2048, 26.4, "5c97ff66d898f5a1.json:193"),
        (4096, 47.1, "5c97ff66d898f5a1.json:201")]),
    (4096, 256, "b_shuffled", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_n4096_k256", [
        (64, 4.33, "f15fac0a07c83b80.json:153"), (128, 4.35, "f15fac0a07c83b80.json:161"),
        (256, 4.34, "f15fac0a07c83b80.json:169"), (512, 4.3, "f15fac0a07c83b80.json:177"),
        (1024, 5.88, "f15fac0a07c83b80.json:185"), (2048, 6.18, "f15fac0a07c83b80.json:193"),
        (4096, 12.2, "f15fac0a07c83b80.json:201")]),
    (4096, 4096, "b_shuffled", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_n4096_k4096", [
        (64, 7.1, "78e6bbcadf087b68.json:153"), (128, 9.09, "78e6bbcadf087b68.json:161"),
        (256, 11.9, "78e6bbcadf087b68.json:169"), (512, 16.5, "78e6bbcadf087b68.json:177"),
        (1024, 23.1, "78e6bbcadf087b68.json:185"), (2048, 39.3, "78e6bbcadf087b68.json:193"),
        (4096, 73.4, "78e6bbcadf087b68.json:201")]),
    (4096, 512, "b_shuffled", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_n4096_k512", [
        (64, 4.48, "a3a340bda94329c4.json:153"), (128, 4.56, "a3a340bda94329c4.json:161"),
        (256, 4.63, "a3a340bda94329c4.json:169"), (512, 5.86, "a3a340bda94329c4.json:177"),
        (1024, 7.42, "a3a340bda94329c4.json:185"), (2048, 9.75, "a3a340bda94329c4.json:193"),
        (4096, 17.0, "a3a340bda94329c4.json:201")]),
    (4096, 8192, "b_shuffled", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_n4096_k8192", [
        (64, 11.6, "d9ecfacca235649e.json:153"), (128, 14.3, "d9ecfacca235649e.json:161"),
        (256, 18.8, "d9ecfacca235649e.json:169"), (512, 28.2, "d9ecfacca235649e.json:177"),
        (1024, 48.2, "d9ecfacca235649e.json:185"), (2048, 76.5, "d9ecfacca235649e.json:193"),
        (4096, 146.0, "d9ecfacca235649e.json:201")]),
    (512, 4096, "b_shuffled", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_n512_k4096", [
        (64, 4.48, "d38d45d96c0eac1e.json:153"), (128, 5.94, "d38d45d96c0eac1e.json:161"),
        (256, 6.34, "d38d45d96c0eac1e.json:169"), (512, 6.84, "d38d45d96c0eac1e.json:177"),
        (1024, 8.58, "d38d45d96c0eac1e.json:185"), (2048, 11.3, "d38d45d96c0eac1e.json:193"),
        (4096, 16.7, "d38d45d96c0eac1e.json:201")]),
    (7168, 384, "b_shuffled", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_n7168_k384", [
        (64, 4.62, "c4f8eed63e5deff1.json:105"), (128, 4.64, "c4f8eed63e5deff1.json:113")]),
    (8192, 1024, "b_shuffled", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_n8192_k1024", [
        (64, 5.2, "5af76bde5712711d.json:153"), (128, 5.49, "5af76bde5712711d.json:161"),
        (256, 6.23, "5af76bde5712711d.json:169"), (512, 8.96, "5af76bde5712711d.json:177"),
        (1024, 12.5, "5af76bde5712711d.json:185"), (2048, 23.2, "5af76bde5712711d.json:193"),
        (4096, 40.9, "5af76bde5712711d.json:201")]),
    (3072, 1536, "row_major", "triton/gemm_a8w8_blockwise_scaled_n3072_k1536", [
        (64, 4.45, "32cbf89d1446d9ff.json:105"), (128, 4.84, "a27c4f99b94cc9f9.json:105"),
        (256, 6.25, "a66a3e81c97b9c74.json:105"), (1024, 12.4, "fe8b2de984da2c8e.json:105"),
        (2048, 17.2, "9cf51249fe32228f.json:105"), (4096, 25.6, "a93ffba3bd75cf4c.json:105"),
        (6144, 41.1, "d44d4c8a6e72fa10.json:105"), (8192, 48.1, "4a159c69e56742a3.json:105"),
        (8193, 47.0, "bfdae6b023b6fb79.json:105")]),
    (7168, 2048, "row_major", "triton/gemm_a8w8_blockwise_scaled_n7168_k2048", [
        (64, 6.28, "06755ba3ee5eb085.json:105"), (128, 8.18, "1bbf98a368b3fcba.json:105"),
        (256, 11.2, "fee7e092eab87fc5.json:105")]),
    (1024, 4096, "b_shuffled_row_major_a_scale", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_row_major_a_scale_n1024_k4096", [
        (64, 5.2, "f5b24e49c1568873.json:153"), (128, 6.06, "f5b24e49c1568873.json:161"),
        (256, 7.7, "f5b24e49c1568873.json:169"), (512, 9.06, "f5b24e49c1568873.json:177"),
        (1024, 12.1, "f5b24e49c1568873.json:185"), (2048, 15.7, "f5b24e49c1568873.json:193"),
        (4096, 24.8, "f5b24e49c1568873.json:201")]),
    (4096, 256, "b_shuffled_row_major_a_scale", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_row_major_a_scale_n4096_k256", [
        (64, 4.12, "5ca82f252cc497e6.json:153"), (128, 4.14, "5ca82f252cc497e6.json:161"),
        (256, 4.13, "5ca82f252cc497e6.json:169"), (512, 4.3, "5ca82f252cc497e6.json:177"),
        (1024, 4.38, "5ca82f252cc497e6.json:185"), (2048, 7.47, "5ca82f252cc497e6.json:193"),
        (4096, 12.4, "5ca82f252cc497e6.json:201")]),
    (4096, 512, "b_shuffled_row_major_a_scale", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_row_major_a_scale_n4096_k512", [
        (64, 4.67, "d9b93d11ae82adf7.json:153"), (128, 4.73, "d9b93d11ae82adf7.json:161"),
        (256, 4.54, "d9b93d11ae82adf7.json:169"), (512, 4.65, "d9b93d11ae82adf7.json:177"),
        (1024, 6.18, "d9b93d11ae82adf7.json:185"), (2048, 9.4, "d9b93d11ae82adf7.json:193"),
        (4096, 16.0, "d9b93d11ae82adf7.json:201")]),
    (512, 4096, "b_shuffled_row_major_a_scale", "flydsl/gemm_a8w8_blockwise_scaled_b_shuffled_row_major_a_scale_n512_k4096", [
        (64, 4.69, "28f1ec94b60ce6b4.json:153"), (128, 5.12, "28f1ec94b60ce6b4.json:161"),
        (256, 7.19, "28f1ec94b60ce6b4.json:169"), (512, 6.78, "28f1ec94b60ce6b4.json:177"),
        (1024, 8.26, "28f1ec94b60ce6b4.json:185"), (2048, 11.8, "28f1ec94b60ce6b4.json:193"),
        (4096, 17.4, "28f1ec94b60ce6b4.json:201")]),
]


def _ref_operands(variant, q, s, b, m, k):
    """(a_scale, b, keyword arguments) of one recorded case: b_shuffled takes aiter's preshuffled b and the
    column-major a_scale; b_shuffled_row_major_a_scale the same b with a K-major a_scale marked
    ``is_row_major``; row_major the row-major b with a K-major a_scale."""
    from aklr_amd import layouts

    if variant == "row_major":
        return s.view(k // 128, m).t().contiguous(), b, {}
    if variant == "b_shuffled_row_major_a_scale":
        sa = s.view(k // 128, m).t().contiguous()
        sa.is_row_major = True
        return sa, layouts.shuffle_weight(b), {"operand_format": "none:preshuffled"}
    return s.view(m, k // 128), layouts.shuffle_weight(b), {"operand_format": "none:preshuffled"}


def reference_all_cases():
    """REFERENCE_ALL as (m, n, k, variant, us, source) cases, in the order of REFERENCE_RECORDED's tuples."""
    return [(m, n, k, variant, us, f"aklr/ops/gemm/impls/{d}/{src}")
            for (n, k, variant, d, pts) in REFERENCE_ALL for (m, us, src) in pts]


REFERENCE_TRACE_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                                    "reference_recorded_fp8_kernel_trace.json")


def reference_recorded_figures(dev, stream, steps=7, cases=None):
    """This build's gemm_a8w8_blockwise_scaled on the shapes the reference records CI times for, each
    call on cold caches (the graph rotates over > 512 MB of operand copies). Beside each event-timed
    figure: the median kernel duration from the committed rocprofv3 kernel trace of
    ``bench.py --probe-reference`` (the kind of figure the reference's tracer records), when present."""
    import aklr_amd
    from aklr_amd import workloads

    try:
        with open(REFERENCE_TRACE_FILE) as f:
            traced = {(r["m"], r["n"], r["k"], r["variant"]): r for r in json.load(f)["shapes"]}
    except (OSError, ValueError, KeyError):
        traced = {}
    out = []
    for (m, n, k, variant, ref_us, src) in (REFERENCE_RECORDED if cases is None else cases):
        copies = []
        for r in range(_copies(gemm8_bytes(m, n, k), lo=2)):
            x = workloads.activations(m, k, seed=300 + r, device=dev)
            q, s = aklr_amd.per_group_quant_fp8(x)
            b, bs = workloads.blockwise_fp8_weight(n, k, seed=400 + r, device=dev)
            sa, bb, kw = _ref_operands(variant, q, s, b, m, k)
            copies.append((q, sa, bb, bs, kw))
            del x

        def run(copies=copies):
            for q, sa, bb, bs, kw in copies:
                aklr_amd.gemm_a8w8_blockwise_scaled(q, bb, sa, bs, **kw)
        g = _capture(run, stream)
        t = _replay_median_ms(g, steps, 1, stream) / len(copies) * 1e3  # median, as the reference reports
        del g, copies
        tf = 2.0 * m * n * k / (t * 1e-6) / 1e12
        out.append({"m": m, "n": n, "k": k, "variant": variant, "us": round(t, 2), "reference_us": ref_us,
                    "speedup": round(ref_us / t, 3), "tflops": round(tf, 1),
                    "gbs": round(gemm8_bytes(m, n, k) / (t * 1e-6) / 1e9, 1), "reference_source": src})
        tr = traced.get((m, n, k, variant))
        if tr is not None:
            out[-1].update(kernel_trace_us=tr["kernel_us"], speedup_kernel_trace=round(ref_us / tr["kernel_us"], 3))
        torch.cuda.empty_cache()
    return out


def mxfp4_figures(dev, stream, steps=10):
    import aklr_amd
    from aklr_amd import layouts, workloads

    out = []
    for m in workloads.MXFP4_M:  # m <= 32 reported against HBM, m >= 512 against the MXFP4 MFMA peak
        for (n, k) in workloads.LLAMA70B_NK:
            # every call on cold operands: rotating (activation, weight) copies of > 512 MB in all
            copies = []
            for r in range(_copies(gemm4_bytes(m, n, k), lo=2)):
                x = workloads.activations(m, k, seed=1 + r, device=dev)
                qa, sa = aklr_amd.dynamic_mxfp4_quant(x, shuffle=True)
                wb, sb = workloads.mxfp4_weight(n, k, seed=10 + r, device=dev)
                copies.append((qa, sa, layouts.shuffle_weight(wb), layouts.e8m0_scales(sb)))
                del x, wb

            def run(copies=copies):
                for qa, sa, wb, sb in copies:
                    aklr_amd.gemm_a4w4_mxfp4(qa, wb, sa, sb)

            g = _capture(run, stream)
            if m <= 32:
                t = _replay_time_ms([g], steps, 2, stream) / len(copies)
            else:  # compute-bound: after the clocks settle, as the FP8 prefill figures
                t = _replay_median_ms(g, steps, 2, stream) / len(copies)
            del g
            rec = {"m": m, "n": n, "k": k, "us": round(t * 1e3, 2)}
            if m <= 32:
                gbs = gemm4_bytes(m, n, k) / (t * 1e-3) / 1e9
                rec.update(gbs=round(gbs, 1), frac_hbm_peak=round(gbs / HBM_PEAK_GBS, 4))
            else:
                tf = 2.0 * m * n * k / (t * 1e-3) / 1e12
                rec.update(tflops=round(tf, 1), frac_mxfp4_peak=round(tf / MXFP4_PEAK_TFLOPS, 4))
            out.append(rec)
            del copies
    return out


# The reference's recorded quantizer times (BASELINE: graph replay with a 1 GiB cache flush per call).
QUANT_REFERENCE_US = {("fp8_1x128", 16384): 55.2, ("fp8_1x128", 2048): 9.43, ("mxfp8", 16384): 51.1}


def quant_figures(dev, stream, steps=20):
    """Rows a1/a4/a5: the three activation quantizers at H=7168, T in {2048, 16384}, called through the C
    ABI on rotating input/output sets of at least 512 MB in all, so the 256 MB last-level cache holds none
    of them (cold, as the reference times them)."""
    from aklr_amd import _lib, workloads

    lib = _lib.lib()
    h = 7168
    out = []
    for t in (2048, 16384):
        n = max(4, -(-(512 << 20) // (t * h * 3)))
        xs = [workloads.activations(t, h, seed=s % 4, device=dev) for s in range(n)]
        q8 = [torch.empty((t, h), dtype=torch.uint8, device=dev) for _ in range(n)]
        s8 = [torch.empty((h // 128, t), dtype=torch.float32, device=dev) for _ in range(n)]
        sm = [torch.empty((t, h // 32), dtype=torch.uint8, device=dev) for _ in range(n)]
        q4 = [torch.empty((t, h // 2), dtype=torch.uint8, device=dev) for _ in range(n)]
        s4 = [torch.empty(((t + 255) // 256 * 256) * ((h // 32 + 7) // 8 * 8), dtype=torch.uint8, device=dev)
              for _ in range(n)]
        st = stream.cuda_stream
        cases = (
            ("fp8_1x128", lambda i: lib.aklr_per_group_quant_fp8(xs[i].data_ptr(), h, q8[i].data_ptr(),
                                                                 s8[i].data_ptr(), t, h, st), 3.03125),
            ("mxfp8", lambda i: lib.aklr_per_group_quant_mxfp8(xs[i].data_ptr(), h, q8[i].data_ptr(),
                                                               sm[i].data_ptr(), t, h, st), 3.03125),
            ("mxfp4", lambda i: lib.aklr_dynamic_mxfp4_quant(xs[i].data_ptr(), h, q4[i].data_ptr(), s4[i].data_ptr(),
                                                             t, h, 1, st), 2.53125),
        )
        for name, fn, bpe in cases:
            def run(fn=fn):
                for i in range(n):
                    fn(i)

            g = _capture(run, stream)
            ms = _replay_time_ms([g], steps, 3, stream) / n
            gbs = t * h * bpe / (ms * 1e-3) / 1e9
            rec = {"kernel": name, "tokens": t, "hidden": h, "us": round(ms * 1e3, 2), "gbs": round(gbs, 1),
                   "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
            ref = QUANT_REFERENCE_US.get((name, t))
            if ref is not None:
                rec["reference_us"] = ref
            out.append(rec)
            del g
        del xs, q8, s8, sm, q4, s4
    return out


def moe_figures(dev, steps=10):
    """Config 5: the experts of the grouped MoE on Zipf(1.1) routing (8 distinct routed experts per
    token plus the shared one), per call, from HIP events over back-to-back calls: after >= 50 ms of
    warm-up calls, the median of 5 windows of steps / 5 calls."""
    import aklr_amd

    e, d, inter, topk = 256, 7168, 2048, 8
    g = torch.Generator(device=dev)
    g.manual_seed(0)

    def fp8(shape):  # finite e4m3 codes
        return torch.randint(0, 0x7E, shape, dtype=torch.uint8, device=dev, generator=g).view(torch.float8_e4m3fn)

    w1, w2 = fp8((e + 1, 2 * inter, d)), fp8((e + 1, d, inter))
    s1 = torch.rand((e + 1, 2 * inter // 128, d // 128), device=dev, generator=g) * 1e-3
    s2 = torch.rand((e + 1, d // 128, inter // 128), device=dev, generator=g) * 1e-3
    p = (1.0 / torch.arange(1, e + 1, device=dev, dtype=torch.float64) ** 1.1).float()
    out = []
    for t in (64, 4096):
        x = torch.randn((t, d), device=dev, generator=g).to(torch.bfloat16)
        ids = torch.multinomial(p.expand(t, e), topk, replacement=False, generator=g).to(torch.int32)
        ids = torch.cat([ids, torch.full((t, 1), e, dtype=torch.int32, device=dev)], 1)
        wts = torch.rand((t, topk + 1), device=dev, generator=g)
        touched = int(torch.unique(ids).numel())
        # at least 50 ms of calls first (the clocks settle under sustained load), then the median of 5
        # windows of back-to-back calls
        t0, n = time.perf_counter(), 0
        while n < 2 or (time.perf_counter() - t0) * 1e3 < 50.0:
            aklr_amd.moe_fp8_experts(x, w1, w2, wts, ids, s1, s2)
            n += 1
            if n % 4 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        per = max(1, steps // 5)
        windows = []
        for _ in range(5):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(per):
                aklr_amd.moe_fp8_experts(x, w1, w2, wts, ids, s1, s2)
            end.record()
            end.synchronize()
            windows.append(start.elapsed_time(end) / per)
        sec = sorted(windows)[2] * 1e-3
        wbytes = touched * (2 * inter * d + d * inter)
        flops = 2 * t * (topk + 1) * (2 * inter * d + d * inter)
        out.append({"tokens": t, "ms": round(sec * 1e3, 3), "experts_touched": touched,
                    "touched_weight_gb": round(wbytes / 1e9, 3),
                    "gbs": round(wbytes / sec / 1e9, 1), "frac_hbm_peak": round(wbytes / sec / 1e9 / HBM_PEAK_GBS, 4),
                    "tflops": round(flops / sec / 1e12, 1), "frac_fp8_peak": round(flops / sec / 1e12 / FP8_PEAK_TFLOPS, 4)})
    del w1, w2
    return out


def decode_floor_figures(dev, stream, weights=None, steps=20):
    """What a kernel that only reads a decode GEMM's bytes takes on this GPU, timed exactly as the GEMMs
    are (back-to-back launches in one graph over rotating buffers of > 512 MB, HIP events on the launch
    stream): the calibration kernel aklr_probe_hbm_read (16-byte non-temporal loads, the best of 256,
    512 and 1024 workgroups with 4 or 8 loads a lane in flight) on the M=1 algorithmic bytes of each
    DeepSeek-V3 decode shape, an empty kernel (the launch floor), and the GEMM at M=1 and M=16 next
    to them."""
    from aklr_amd import _lib, workloads

    lib = _lib.lib()
    st = stream.cuda_stream
    sink = torch.empty(1024 * 256, dtype=torch.int32, device=dev)
    empty = torch.empty(16, dtype=torch.uint8, device=dev)

    def launches(fn, count):
        g = _capture(lambda: [fn() for _ in range(count)], stream)
        t = _replay_time_ms([g], steps, 2, stream) / count
        del g
        return t

    out = {"empty_kernel_us": round(launches(lambda: lib.aklr_probe_hbm_read(empty.data_ptr(), 0, sink.data_ptr(),
                                                                             256, 4, st), 32) * 1e3, 2),
           "shapes": []}
    for (n, k) in workloads.DEEPSEEK_NK:
        nbytes = gemm8_bytes(1, n, k)
        bufs = [torch.empty((nbytes + 15) // 16 * 16, dtype=torch.uint8, device=dev).fill_(1)
                for _ in range(_copies(nbytes, lo=4))]
        best = None
        for wg in (256, 512, 1024):
            for unroll in (4, 8):
                def run(wg=wg, unroll=unroll):
                    for b in bufs:
                        lib.aklr_probe_hbm_read(b.data_ptr(), nbytes, sink.data_ptr(), wg, unroll, st)

                g = _capture(run, stream)
                t = _replay_time_ms([g], steps, 2, stream) / len(bufs)
                del g
                if best is None or t < best[0]:
                    best = (t, wg, unroll)
        rec = {"n": n, "k": k, "bytes": nbytes, "read_us": round(best[0] * 1e3, 2),
               "read_gbs": round(nbytes / (best[0] * 1e-3) / 1e9, 1), "read_workgroups": best[1],
               "read_unroll": best[2]}
        del bufs
        if weights is not None:
            for m in (1, 16):
                t = time_gemm8(dev, m, n, k, weights, steps, stream)
                rec[f"gemm_m{m}_us"] = round(t * 1e3, 2)
                rec[f"gemm_m{m}_vs_read"] = round(best[0] / t, 3)
        out["shapes"].append(rec)
        torch.cuda.empty_cache()
    return out


def probe_prefill(dev, stream, calls=6):
    """The program the prefill counters are read on: the FP8 prefill GEMM at M=4096 on the three
    DeepSeek-V3 shapes (the 192x192, 256x256 and 256x224 LDS plans), each called ``calls`` times on
    rotating cold operand copies, after one warm-up call per copy."""
    import aklr_amd
    from aklr_amd import layouts, workloads

    m = 4096
    plan = []
    for (n, k) in workloads.DEEPSEEK_NK:
        copies = []
        for r in range(_copies(gemm8_bytes(m, n, k), lo=2)):
            x = workloads.activations(m, k, seed=1 + r, device=dev)
            q, s = aklr_amd.per_group_quant_fp8(x)
            b, bs = workloads.blockwise_fp8_weight(n, k, seed=2 + r, device=dev)
            copies.append((q, s.view(m, k // 128), layouts.shuffle_weight(b), bs))
            del x, b
        for i in range(len(copies) + calls):
            q, s, b, bs = copies[i % len(copies)]
            aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s, bs, operand_format="none:preshuffled")
        torch.cuda.synchronize()
        print(f"[bench] prefill probe m={m} n={n} k={k}: {len(copies) + calls} calls", file=sys.stderr, flush=True)
        plan.append({"case": "fp8_lds_m4096", "m": m, "n": n, "k": k, "kernels": ["gemm8_lds_kernel"],
                     "launches": len(copies) + calls, "warm": len(copies)})
        del copies
        torch.cuda.empty_cache()
    _calibration_copy(dev)
    print("[bench] probe plan " + json.dumps(plan), file=sys.stderr, flush=True)


def _calibration_copy(dev):
    """A plain 256 MiB device copy, three times: what FETCH_SIZE and WRITE_SIZE read for 268,435,456
    bytes moved scales the GEMMs' readings in the same profiler run."""
    src = torch.empty(256 * 2**20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    print("[bench] calibration copy: 3 x 268435456 bytes", file=sys.stderr, flush=True)


def probe_counters(dev, stream, calls=4):
    """The program the per-kernel counter summaries are read on (rocprofv3 --pmc / --kernel-trace). Every
    case runs its GEMM once per rotating cold operand copy (> 512 MB in all) and then ``calls`` more
    times; the calibration copy ends the run. Cases, in launch order:
      fp8_lds_m1024      FP8 LDS kernel, M=1024 on the three DeepSeek-V3 shapes
      fp8_stream_m64/128 FP8 stream kernel at M=64 and 128 on the DeepSeek-V3 shapes and on 7168x2048
      mxfp4_lds          MXFP4 LDS kernel at M=512 and 4096 on the three Llama-3-70B shapes
      moe_t4096          the grouped MoE experts at T=4096 (Zipf(1.1) top-8 + shared; the gate-up and
                         the down launch are moe_gemm_kernel<true, ...> and <false, ...>)
    A JSON line on stderr lists each case with its kernel-name patterns and its number of launches of each
    (the MoE's gate-up and down launches alternate), in order, so a parser can assign the profiler's
    dispatches to cases."""
    import aklr_amd
    from aklr_amd import layouts, workloads

    plan = []

    def fp8_case(tag, m, n, k, kernel):
        copies = []
        for r in range(_copies(gemm8_bytes(m, n, k), lo=2)):
            x = workloads.activations(m, k, seed=1 + r, device=dev)
            q, s = aklr_amd.per_group_quant_fp8(x)
            b, bs = workloads.blockwise_fp8_weight(n, k, seed=2 + r, device=dev)
            copies.append((q, s.view(m, k // 128), layouts.shuffle_weight(b), bs))
            del x, b
        torch.cuda.synchronize()
        for i in range(len(copies) + calls):
            q, s, b, bs = copies[i % len(copies)]
            aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s, bs, operand_format="none:preshuffled")
        torch.cuda.synchronize()
        plan.append({"case": tag, "m": m, "n": n, "k": k, "kernels": [kernel], "launches": len(copies) + calls,
                     "warm": len(copies)})
        print(f"[bench] counters probe {tag} m={m} n={n} k={k}", file=sys.stderr, flush=True)
        del copies
        torch.cuda.empty_cache()

    for (n, k) in workloads.DEEPSEEK_NK:
        fp8_case("fp8_lds_m1024", 1024, n, k, "gemm8_lds_kernel")
    for m in (64, 128):
        for (n, k) in workloads.DEEPSEEK_NK + ((7168, 2048),):
            fp8_case(f"fp8_stream_m{m}", m, n, k, "gemm8_stream_kernel")

    for m in (512, 4096):
        for (n, k) in workloads.LLAMA70B_NK:
            copies = []
            for r in range(_copies(gemm4_bytes(m, n, k), lo=2)):
                x = workloads.activations(m, k, seed=1 + r, device=dev)
                qa, sa = aklr_amd.dynamic_mxfp4_quant(x, shuffle=True)
                wb, sb = workloads.mxfp4_weight(n, k, seed=10 + r, device=dev)
                copies.append((qa, sa, layouts.shuffle_weight(wb), layouts.e8m0_scales(sb)))
                del x, wb
            torch.cuda.synchronize()
            for i in range(len(copies) + calls):
                qa, sa, wb, sb = copies[i % len(copies)]
                aklr_amd.gemm_a4w4_mxfp4(qa, wb, sa, sb)
            torch.cuda.synchronize()
            plan.append({"case": "mxfp4_lds", "m": m, "n": n, "k": k, "kernels": ["gemm4_lds_kernel"],
                         "launches": len(copies) + calls, "warm": len(copies)})
            print(f"[bench] counters probe mxfp4 m={m} n={n} k={k}", file=sys.stderr, flush=True)
            del copies
            torch.cuda.empty_cache()

    e, d, inter, topk, t = 256, 7168, 2048, 8, 4096
    w1, s1 = workloads.moe_expert_weights(e + 1, 2 * inter, d, seed=20, device=dev)
    w2, s2 = workloads.moe_expert_weights(e + 1, d, inter, seed=21, device=dev)
    x = workloads.activations(t, d, seed=22, device=dev, outliers=False)
    ids, wts = workloads.moe_routing(t, e, topk, seed=23, device=dev)
    moe_calls = 1 + calls
    for _ in range(moe_calls):
        aklr_amd.moe_fp8_experts(x, w1, w2, wts, ids, s1, s2)
    torch.cuda.synchronize()
    plan.append({"case": "moe_t4096", "tokens": t, "kernels": ["moe_gemm_kernel<0,", "moe_gemm_kernel<1,"],
                 "launches": moe_calls, "warm": 1})
    print("[bench] counters probe moe t=4096", file=sys.stderr, flush=True)
    del w1, w2, s1, s2
    torch.cuda.empty_cache()
    _calibration_copy(dev)
    print("[bench] probe plan " + json.dumps(plan), file=sys.stderr, flush=True)


def probe_reference(dev, stream, calls=5, cases=None):
    """The program the kernel-trace comparison with the reference's recorded times is read on: this
    build's FP8 GEMM on each of the reference's recorded shapes (the 17 of REFERENCE_RECORDED, or the
    given cases), once per rotating cold operand copy and then ``calls`` more times (rocprofv3
    --kernel-trace gives each launch's duration, the kind of figure the reference's own tracer records)."""
    import aklr_amd
    from aklr_amd import workloads

    plan = []
    for (m, n, k, variant, ref_us, src) in (REFERENCE_RECORDED if cases is None else cases):
        copies = []
        for r in range(_copies(gemm8_bytes(m, n, k), lo=2)):
            x = workloads.activations(m, k, seed=300 + r, device=dev)
            q, s = aklr_amd.per_group_quant_fp8(x)
            b, bs = workloads.blockwise_fp8_weight(n, k, seed=400 + r, device=dev)
            sa, bb, kw = _ref_operands(variant, q, s, b, m, k)
            copies.append((q, sa, bb, bs, kw))
            del x, b
        torch.cuda.synchronize()
        for i in range(len(copies) + calls):
            q, sa, bb, bs, kw = copies[i % len(copies)]
            aklr_amd.gemm_a8w8_blockwise_scaled(q, bb, sa, bs, **kw)
        torch.cuda.synchronize()
        plan.append({"case": f"{m}x{n}x{k} {variant}", "m": m, "n": n, "k": k, "variant": variant,
                     "reference_us": ref_us, "kernels": ["gemm8_"], "launches": len(copies) + calls,
                     "warm": len(copies)})
        del copies
        torch.cuda.empty_cache()
    print("[bench] probe plan " + json.dumps(plan), file=sys.stderr, flush=True)


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "gemm8_stream_m16_n7168_k16384_traffic.json")


def probe_traffic(dev, stream):
    """The program the traffic counters are read on: the dominant decode GEMM (M=16, N=7168,
    K=16384, preshuffled weights, 8 rotating copies, 3 rounds), then a plain 256 MiB copy three times
    (the calibration: its FETCH_SIZE and WRITE_SIZE should read 256 MiB each)."""
    import aklr_amd
    from aklr_amd import layouts, workloads

    m, n, k = 16, 7168, 16384
    x = workloads.activations(m, k, seed=5, device=dev)
    q, s = aklr_amd.per_group_quant_fp8(x)
    copies = []
    for r in range(8):
        b, bs = workloads.blockwise_fp8_weight(n, k, seed=100 + r, device=dev)
        copies.append((layouts.shuffle_weight(b), bs))
    for _ in range(3):
        for b, bs in copies:
            aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s.view(m, k // 128), bs, operand_format="none:preshuffled")
    _calibration_copy(dev)
    print("[bench] probe plan " + json.dumps([{"case": "fp8_stream_m16", "m": m, "n": n, "k": k,
                                               "kernels": ["gemm8_stream_kernel"], "launches": 24, "warm": 0}]),
          file=sys.stderr, flush=True)
    print("[bench] traffic probe done", file=sys.stderr, flush=True)


def load_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def cpu_baseline():
    """The CPU oracle on one whole decode step (the 15 quantize-then-GEMM pairs: quantize, dequantize,
    fp32 matmul), the median of 3 timed repetitions after a warm-up one."""
    import numpy as np

    from aklr_amd import workloads
    from oracle import gemm as ogemm
    from oracle import quant as oquant

    cases = []
    for (n, k) in workloads.DEEPSEEK_NK:
        b, bs = workloads.blockwise_fp8_weight(n, k, seed=4, device="cpu")
        b, bs = b.view(torch.uint8).numpy(), bs.numpy()
        for m in workloads.DECODE_M:
            x = workloads.activations(m, k, seed=3 + m, device="cpu")
            cases.append((x.view(torch.int16).numpy().view(np.uint16), b, bs, m, n, k))
    total_bytes = sum(gemm8_bytes(m, n, k) + quant8_bytes(m, k) for _, _, _, m, n, k in cases)

    def step():
        for xb, b, bs, m, n, k in cases:
            q, s = oquant.per_group_quant_fp8(xb)
            ogemm.gemm_a8w8_blockwise_scaled(q, b, s, bs, scale_major_mode="MN")

    step()
    reps = []
    for _ in range(3):
        t0 = time.perf_counter()
        step()
        reps.append(time.perf_counter() - t0)
    dt = sorted(reps)[1]
    try:
        from threadpoolctl import threadpool_info

        cores = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
    except Exception:  # noqa: BLE001
        cores = os.cpu_count() or 1
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), None)
    except OSError:
        pass
    return {
        "value": round(total_bytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": int(cores),
        "cpu_count": os.cpu_count(),
        "torch_threads": torch.get_num_threads(),
        "cpu_model": model,
        "kind": "port",
        "sample": f"one decode step, M in {{1,4,16,64,128}} x (N,K) in (2112,7168),(24576,1536),(7168,16384): "
                  f"quant + dequant + fp32 matmul, median of 3 reps ({', '.join(f'{r:.2f}' for r in reps)} s)",
    }


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layout", choices=("preshuffled", "row_major"), default="preshuffled")
    ap.add_argument("--no-extras", action="store_true", help="skip the prefill/MXFP4 figures")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--probe-traffic", action="store_true",
                    help="only run the dominant kernel and a calibration copy (for rocprofv3 --pmc)")
    ap.add_argument("--probe-prefill", action="store_true",
                    help="only run the FP8 prefill GEMM at M=4096 on the three shapes (for rocprofv3 --pmc)")
    ap.add_argument("--probe-floor", action="store_true",
                    help="only time the decode floors: an empty kernel and a pure HBM read of each decode "
                         "shape's bytes, beside the GEMM (for rocprofv3 --kernel-trace)")
    ap.add_argument("--probe-counters", action="store_true",
                    help="only run the per-kernel counter cases (FP8 LDS at M=1024, FP8 stream at M=64/128, "
                         "MXFP4 LDS at M=512/4096, MoE at T=4096) and a calibration copy (for rocprofv3 --pmc)")
    ap.add_argument("--probe-reference", action="store_true",
                    help="only run the FP8 GEMM on the reference's 17 recorded shapes (for rocprofv3 "
                         "--kernel-trace)")
    ap.add_argument("--probe-reference-all", action="store_true",
                    help="the same on every point the reference records at m >= 64 (REFERENCE_ALL)")
    ap.add_argument("--reference-all", action="store_true",
                    help="only time every point of REFERENCE_ALL as the default run times the 17 (HIP "
                         "events) and print one JSON line")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    # graphs are captured on (and every launch and event goes to) one non-default stream of
    # default priority
    stream = torch.cuda.Stream(dev)
    torch.cuda.set_stream(stream)
    if args.probe_traffic:
        probe_traffic(dev, stream)
        return 0
    if args.probe_prefill:
        probe_prefill(dev, stream)
        return 0
    if args.probe_counters:
        probe_counters(dev, stream)
        return 0
    if args.probe_reference or args.probe_reference_all:
        probe_reference(dev, stream, cases=reference_all_cases() if args.probe_reference_all else None)
        return 0
    if args.reference_all:
        rows = []
        for case in reference_all_cases():  # one at a time, each printed as it ends
            rows += reference_recorded_figures(dev, stream, cases=[case])
            r = rows[-1]
            print(f"[bench] {r['m']} x {r['n']} x {r['k']} {r['variant']}: {r['us']} us, reference "
                  f"{r['reference_us']} us", file=sys.stderr, flush=True)
        ratios = [r["speedup"] for r in rows]
        geo = math.exp(sum(math.log(x) for x in ratios) / len(ratios))
        print(json.dumps({"reference_all": rows, "points": len(rows), "geomean_reference_over_this": round(geo, 3),
                          "points_below_0.8": sum(x < 0.8 for x in ratios),
                          "points_at_or_above_1.0": sum(x >= 1.0 for x in ratios)}), flush=True)
        return 0
    if args.probe_floor:
        step_fn, n_sets, step_bytes, weights, xs = build_decode(dev, True)
        print(json.dumps(decode_floor_figures(dev, stream, weights)), flush=True)
        return 0
    shuffled = args.layout == "preshuffled"
    print(f"[bench] building decode workload ({args.layout})", file=sys.stderr, flush=True)
    step_fn, n_sets, step_bytes, weights, xs = build_decode(dev, shuffled)
    copies_per_shape = {nk: len(c) for nk, c in weights.items()}
    graphs = [_capture(step_fn(r), stream) for r in range(n_sets)]
    print(f"[bench] {len(graphs)} step graphs captured; timing {args.steps} steps", file=sys.stderr, flush=True)
    ms_per_step = _replay_time_ms(graphs, args.steps, args.warmup, stream)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    del graphs
    fused_fn = fused_step_fn(weights, xs, shuffled)
    graphs = [_capture(fused_fn(r), stream) for r in range(n_sets)]
    ms_fused = _replay_time_ms(graphs, args.steps, args.warmup, stream)
    print(f"[bench] decode step {ms_per_step:.4f} ms, with the fused quantization {ms_fused:.4f} ms",
          file=sys.stderr, flush=True)

    m_dom, n_dom, k_dom = 16, 7168, 16384
    t_dom = time_gemm8(dev, m_dom, n_dom, k_dom, weights, max(10, args.steps), stream, shuffled)
    dom_bytes = gemm8_bytes(m_dom, n_dom, k_dom)
    achieved = dom_bytes / (t_dom * 1e-3) / 1e9
    per_shape = []
    for (n, k) in ((2112, 7168), (24576, 1536), (7168, 16384)):
        for m in (1, 16, 64, 128):
            t = time_gemm8(dev, m, n, k, weights, 10, stream, shuffled)
            per_shape.append({"m": m, "n": n, "k": k, "us": round(t * 1e3, 2),
                              "gbs": round(gemm8_bytes(m, n, k) / (t * 1e-3) / 1e9, 1)})
    floor = decode_floor_figures(dev, stream)
    del graphs, weights
    torch.cuda.empty_cache()

    extras = {"decode_fused_quant": {"ms_per_step": round(ms_fused, 4),
                                     "speedup_vs_two_ops": round(ms_per_step / ms_fused, 3)},
              "decode_floor": floor}
    if not args.no_extras:
        print("[bench] prefill and MXFP4 figures", file=sys.stderr, flush=True)
        extras["prefill_fp8"] = prefill_figures(dev, stream)
        torch.cuda.empty_cache()
        extras["reference_recorded_fp8"] = reference_recorded_figures(dev, stream)
        torch.cuda.empty_cache()
        extras["mxfp4"] = mxfp4_figures(dev, stream)
        torch.cuda.empty_cache()
        extras["quant"] = quant_figures(dev, stream)
        torch.cuda.empty_cache()
        print("[bench] MoE (config 5) figures", file=sys.stderr, flush=True)
        extras["moe_fp8_deepseek_v3"] = moe_figures(dev)
        torch.cuda.empty_cache()
    cpu = None
    if not args.no_cpu:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline()

    traffic = load_traffic()
    le16 = {}
    for r in per_shape:
        if r["m"] <= 16:
            le16.setdefault(f"{r['n']}x{r['k']}", {})[f"m{r['m']}"] = round(r["gbs"] / HBM_PEAK_GBS, 3)
    line = {
        "metric": "block-scaled FP8 GEMM decode HBM GB/s (DeepSeek-V3 decode config)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3",
        "data": "synthetic (seeded N(0,1) activations with 1% x20 outliers, N(0,0.02) weights)",
        "config": {
            "workload": "deepseek_v3_decode_fp8_blockscale: M in {1,4,16,64,128} x (N,K) in "
                        "{(2112,7168),(24576,1536),(7168,16384)}, quant + GEMM per step",
            "b_layout": args.layout,
            "weight_copies_per_shape": {f"{n}x{k}": c for (n, k), c in copies_per_shape.items()},
            "step_graphs": n_sets,
            "step_bytes": step_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"gemm8_stream_kernel (M={m_dom}, N={n_dom}, K={k_dom})",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": (traffic or {}).get("bytes_per_launch"),
            "traffic_source": (traffic or {}).get("source"),
            "launch_us": round(t_dom * 1e3, 2),
            "bytes_per_launch": dom_bytes,
            # the north star's decode target (0.70 of HBM at M <= 16), per (N, K): each GEMM's fraction
            "decode_m_le16_frac_hbm": le16,
        },
        "decode_per_shape": per_shape,
        **extras,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
