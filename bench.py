"""W4A8 decode-GEMV sweep benchmark on one MI355X.

One step = the W4A8 quantized linear (per-token fp8 act-quant + int4 x fp8 GEMM, bf16 out) at the
four Llama-3-8B layer shapes (qkv 4096x6144, o_proj 4096x4096, gate_up 4096x28672, down 14336x4096)
for every M in {1, 2, 4, 8, 16}: 20 calls, captured once into a HIP graph and replayed. Weights are
GPTQ-symmetric int4 group 128 with fp16 scales |N(0, 0.02)|, activations bf16 N(0,1) with 0.1% of
channels x50; 5 copies of the weight set are cycled (each M uses its own copy, 555 MB of weights
per step) so no step re-reads weights out of the 256 MB Infinity Cache.

value = algorithmic bytes of the step (codes N*K/2 + fp16 scales + bf16 x in + bf16 out) x steps /
wall time, with everything resident in HBM. The roofline object is the decode GEMV kernel alone at
the largest shape (gate_up, M=1, one launch per call): algorithmic bytes per launch / mean launch
time from HIP events on the launch stream, against 8 TB/s. decode_per_shape times every call of the
step on its own (GB/s and fraction per shape and M). cpu_baseline is the reference's
dequantize-then-matmul CPU path (oracle/baseline.py): the whole sweep step on all host cores, median
of 5 passes, with the CPU model, rank 0 only. prefill_config3 is configs[2]/[3]: every shape at
M = 512, 2048, 8192 on the producer pair (act-quant outside the timed region).

other_configs reports the remaining BASELINE configs through the same operator API: cfg1 (AWQ
zero-point int4, M=16, K=2560, N=9728), cfg4 (MoE E=128 top-8 H=2048 I=768, T in {1,16,256,4096})
and cfg5 (MXFP4 E8M0, K x N in {8192x28672, 28672x8192}, M in {1,16,4096}); GB/s against 8 TB/s
for the decode sizes, TFLOPS against the 5 PFLOPS fp8 peak for the large ones.

next_formats reports the W4A16 arm (unquantized activations) and NVFP4 through the same operator
API (not BASELINE configs; the shapes are the gate_up ones above).

producer_norm_step times the same sweep with its inputs coming out of the RMSNorm + residual-add
producer: once with the linear quantizing its bf16 input, once with the producer's fp8 pair
(no act-quant launches).

Modes for profiling runs (same committed file): --read-floor times the streaming-read floor of one
launch at the decode weight sizes, --profile-kernel runs only the roofline loop,
--profile-prefill FMT M K N times one prefill GEMM, --copy-calib runs a plain device copy of known
size (for scaling rocprofv3 byte counters).
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for p in (str(REPO), str(REPO / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

SHAPES = [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)]  # (K, N)
MS = [1, 2, 4, 8, 16]
GROUP = 128
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
METRIC = "W4A8 GEMM HBM GB/s (M<=16) and TFLOPS (M>=2048), % roofline, 1 MI355X"


def algo_bytes(M: int, K: int, N: int) -> int:
    return N * K // 2 + (K // GROUP) * N * 2 + M * K * 2 + M * N * 2


def make_weights(kernels, K: int, N: int, gen, dev):
    import torch

    codes = torch.randint(0, 16, (N, K), generator=gen, device=dev, dtype=torch.int32)
    sh = torch.arange(0, 32, 4, dtype=torch.int32, device=dev)
    w = (codes.view(N, K // 8, 8) << sh).sum(-1, dtype=torch.int32)
    del codes
    s = (torch.randn(K // GROUP, N, generator=gen, device=dev).abs() * 0.02).to(torch.float16)
    tiles = kernels.repack_w4(w)
    del w
    return tiles, s


def make_x(M: int, K: int, seed: int, dev):
    import synth

    return synth.activations(M, K, seed=seed, outliers=True).to(dev)


def cpu_baseline_leg() -> dict:
    from oracle import baseline

    r = baseline.run(SHAPES, MS, GROUP, seed=1, repeats=5)
    gbs = r["bytes"] / r["seconds"] / 1e9
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": r["cores"], "kind": "port",
            "cpu_model": r["cpu_model"],
            "median_of": r["repeats"], "seconds_per_pass": r["all_seconds"],
            "dequant_s": round(r["dequant_s"], 4), "matmul_s": round(r["matmul_s"], 4),
            "total_s": round(r["seconds"], 4),
            "sample": f"one full sweep step (4 Llama-3-8B shapes x M in {{1,2,4,8,16}}), {r['bytes'] / 1e6:.0f} MB "
                      f"algorithmic, timed {r['repeats']} times (median pass reported); per call: per-token e4m3 "
                      f"round trip + int4 dequant to f32 + f32 matmul; torch CPU, {r['cores']} threads"}


def roofline_leg(kernels, dev, reps: int = 60) -> dict:
    """Mean launch time of the decode GEMV at gate_up (K=4096, N=28672), M=1, bf16 input quantized
    in the kernel's prologue (the product's decode path: one launch per call), cycling 10 weight
    copies (590 MB, over twice the 256 MB MALL) so every launch streams from HBM. The launches
    queue up behind a GPU sleep and run back to back; one event pair on the launching stream
    brackets them, so the mean is kernel time plus the back-to-back dispatch gap, as rocprof's
    per-kernel durations are."""
    import torch

    K, N = 4096, 28672
    gen = torch.Generator(device=dev).manual_seed(7)
    copies = [make_weights(kernels, K, N, gen, dev) for _ in range(10)]
    x = make_x(1, K, 70, dev)
    for i in range(10):  # warm
        t, sc = copies[i % 10]
        kernels.w4a8_linear(x, t, sc, None, GROUP)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(100_000_000)  # keep the GPU busy while the launches queue up
    start.record(stream)
    for i in range(reps):
        t, sc = copies[i % 10]
        kernels.w4a8_linear(x, t, sc, None, GROUP)
    end.record(stream)
    torch.cuda.synchronize()
    mean_us = start.elapsed_time(end) * 1e3 / reps
    nbytes = algo_bytes(1, K, N)
    achieved = nbytes / (mean_us * 1e-6) / 1e9
    traffic = None
    tf = REPO / "profiles" / "gemv_gate_up_m1_traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("traffic_bytes_per_launch")
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": "gemv_walk_kernel<1,4,kModeI4,SYM,1,bf16> (strip-walking decode GEMV, int4 sym g128, act quant "
                      "in the row phase, 256 workgroups of two 4-wave sets) K=4096 N=28672 M=1",
            "algorithmic_bytes_per_launch": nbytes, "mean_launch_us": round(mean_us, 3), "launches": reps}


def prefill_leg(kernels, dev) -> dict:
    """TFLOPS of the MFMA GEMM at every configs[2]/[3] shape (M = 512, 2048, 8192), one warm call
    then 5 timed calls on the producer pair (x_fp8, act_scales): the act-quant launch is outside the
    timed region (in_op_quant_us adds it back for one shape per M)."""
    import torch

    out = {"input": "producer pair (x_fp8, act_scales); act-quant outside the timed region"}
    gen = torch.Generator(device=dev).manual_seed(9)
    for K, N in SHAPES:
        tiles, sc = make_weights(kernels, K, N, gen, dev)
        for M in (512, 2048, 8192):
            x = make_x(M, K, 90 + M, dev)
            q, s = kernels.act_quant(x)
            kernels.w4a8_linear(x, tiles, sc, None, GROUP, x_fp8=q, act_scales=s)
            torch.cuda.synchronize()
            reps = 5
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(reps):
                kernels.w4a8_linear(x, tiles, sc, None, GROUP, x_fp8=q, act_scales=s)
            b.record()
            torch.cuda.synchronize()
            us = a.elapsed_time(b) * 1e3 / reps
            tflops = 2.0 * M * N * K / (us * 1e-6) / 1e12
            out[f"{K}x{N}_M{M}"] = {"us": round(us, 1), "tflops": round(tflops, 1),
                                    "frac_fp8_peak": round(tflops / FP8_PEAK_TFLOPS, 4)}
            if (K, N) == (4096, 28672):
                out[f"{K}x{N}_M{M}"]["in_op_quant_us"] = round(
                    _time_calls([lambda: kernels.w4a8_linear(x, tiles, sc, None, GROUP)], 5), 1)
        del tiles, sc
    return out


def decode_shapes_leg(kernels, dev) -> dict:
    """Every configs[1] call on its own: (shape, M) -> mean us per call (act-quant + GEMV, or the
    one fused launch) with back-to-back launches, weights rotated over more than 600 MB (over twice
    the MALL) so every call streams from HBM; GB/s on the algorithmic bytes and the fraction of the
    8 TB/s peak."""
    import torch

    out = {}
    gen = torch.Generator(device=dev).manual_seed(5)
    for K, N in SHAPES:
        wbytes = N * K // 2 + (K // GROUP) * N * 2
        copies = [make_weights(kernels, K, N, gen, dev) for _ in range(max(4, (600 << 20) // wbytes + 1))]
        for M in MS:
            x = make_x(M, K, 100 + M, dev)
            us = _time_calls([lambda c=c: kernels.w4a8_linear(x, c[0], c[1], None, GROUP) for c in copies],
                             max(60, 2 * len(copies)))
            out[f"{K}x{N}_M{M}"] = _gbs(algo_bytes(M, K, N), us)
        del copies
        torch.cuda.empty_cache()
    return out


def profile_prefill(kernels, dev, fmt: str, M: int, K: int, N: int) -> dict:
    """One prefill GEMM shape, 2 warm + 5 timed calls on the producer pair, for counter runs."""
    import torch

    gen = torch.Generator(device=dev).manual_seed(9)
    z = None
    if fmt == "int4":
        tiles, sc = make_weights(kernels, K, N, gen, dev)
        g, e2 = GROUP, False
    elif fmt == "nvfp4":
        tiles = kernels.repack_w4(_rand_words((N, K // 8), gen, dev), weight_is_e2m1=True)
        sc = (torch.rand(K // 16, N, generator=gen, device=dev) * 6 + 0.25).to(torch.float8_e4m3fn)
        z = torch.rand(N, generator=gen, device=dev) * 1e-3 + 1e-4
        g, e2 = 16, True
    else:
        tiles = kernels.repack_w4(_rand_words((N, K // 8), gen, dev), weight_is_e2m1=True)
        sc = torch.randint(119, 128, (K // 32, N), generator=gen, device=dev, dtype=torch.int32).to(torch.uint8)
        g, e2 = 32, True
    x = make_x(M, K, 5, dev)
    q, s = kernels.act_quant(x)
    us = _time_calls([lambda: kernels.w4a8_linear(x, tiles, sc, z, g, weight_is_e2m1=e2, x_fp8=q,
                                                  act_scales=s)], 5)
    return {"profile_prefill": fmt, "M": M, "K": K, "N": N, **_tflops(2.0 * M * N * K, us)}


def profile_moe(kernels, dev, T: int) -> dict:
    """One configs[4] MoE call shape (E=128, top-8, H=2048, I=768, int4 g128), 2 warm + 5 timed
    calls, for kernel-trace and counter runs."""
    import torch

    gen = torch.Generator(device=dev).manual_seed(17)
    E, k, H, I, g = 128, 8, 2048, 768, 128
    w13 = kernels.repack_w4(_rand_words((E, 2 * I, H // 8), gen, dev))
    s13 = (torch.randn(E, H // g, 2 * I, generator=gen, device=dev).abs() * 0.02 + 1e-4).to(torch.float16)
    w2 = kernels.repack_w4(_rand_words((E, H, I // 8), gen, dev))
    s2 = (torch.randn(E, I // g, H, generator=gen, device=dev).abs() * 0.02 + 1e-4).to(torch.float16)
    x = make_x(T, H, 400 + T, dev)
    logits = torch.randn(T, E, generator=gen, device=dev).to(torch.bfloat16)
    us = _time_calls([lambda: kernels.w4a8_moe(x, w13, s13, None, w2, s2, None, logits, k, True)], 5)
    return {"profile_moe": T, "us": round(us, 2)}


def _time_calls(calls, reps: int) -> float:
    """Mean microseconds per call of `reps` calls cycling through `calls`, queued behind a GPU sleep
    and bracketed by one event pair on the launching stream (kernels plus back-to-back gaps)."""
    import torch

    for c in calls[: min(len(calls), 3)]:
        c()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(50_000_000)
    a.record(stream)
    for i in range(reps):
        calls[i % len(calls)]()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / reps


def read_floor(dev) -> dict:
    """The HBM streaming-read floor of one launch (w4a8_probe_read): for each decode call's weight
    size, the fastest of 17 launch shapes of a plain read kernel (one-shot grids of U 16-byte loads per
    thread and T threads per workgroup, persistent grids of G workgroups), 60 back-to-back launches
    over 10 buffer copies (more than the 256 MB MALL) bracketed by one event pair on the launching
    stream, as the decode GEMV's per-call times are taken; plus an empty launch (one 64-thread
    workgroup reading 16 bytes) timed the same way."""
    import torch

    lib = importlib.import_module("minisglang-rdna4_amd._abi").load()
    sizes = {"o_proj M=1 (4096x4096)": 8667136, "qkv M=1 (4096x6144)": 12996608,
             "down M=1 (14336x4096)": 30314496, "gate_up M=1 (4096x28672)": 60620800,
             "MXFP4 M=1 (8192x28672)": 124854272}
    shapes = [(4, 256, 0), (8, 256, 0), (16, 256, 0), (4, 512, 0), (8, 512, 0), (8, 1024, 0), (4, 256, 1024),
              (8, 256, 1024), (8, 512, 512), (8, 512, 1024), (4, 1024, 256), (8, 1024, 256), (4, 1024, 512),
              (8, 256, 2048), (16, 256, 1024), (8, 512, 768), (4, 512, 2048)]
    maxb = max(sizes.values())
    bufs = [torch.full((maxb,), i + 1, dtype=torch.uint8, device=dev) for i in range(10)]
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()
    sptr = stream.cuda_stream

    def timed(launch, reps=60):
        for i in range(10):
            launch(bufs[i % 10])
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(reps):
            launch(bufs[i % 10])
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / reps

    out = {}
    for name, nb in sizes.items():
        best = None
        for u, t, g in shapes:
            us = timed(lambda buf: lib.w4a8_probe_read(buf.data_ptr(), nb, u, t, g, sink.data_ptr(), sptr))
            if best is None or us < best[0]:
                best = (us, f"{'persist' if g else 'oneshot'} U={u} T={t}" + (f" G={g}" if g else ""))
        gbs = nb / (best[0] * 1e-6) / 1e9
        out[name] = {"bytes": nb, "shape": best[1], "us": round(best[0], 2), "GB/s": round(gbs, 1),
                     "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    out["empty launch"] = {"us": round(timed(lambda buf: lib.w4a8_probe_read(buf.data_ptr(), 16, 1, 64, 1,
                                                                             sink.data_ptr(), sptr)), 2)}
    return out


def _rand_words(shape, gen, dev):
    import torch

    return torch.randint(-2**31, 2**31 - 1, shape, generator=gen, device=dev, dtype=torch.int32)


def _gbs(nbytes: int, us: float) -> dict:
    g = nbytes / (us * 1e-6) / 1e9
    return {"us": round(us, 2), "GB/s": round(g, 1), "frac_hbm_peak": round(g / HBM_PEAK_GBS, 4), "bytes": nbytes}


def _tflops(flops: float, us: float) -> dict:
    t = flops / (us * 1e-6) / 1e12
    return {"us": round(us, 1), "TFLOPS": round(t, 1), "frac_fp8_peak": round(t / FP8_PEAK_TFLOPS, 4)}


def configs_leg(kernels, dev) -> dict:
    """The other BASELINE configs through the product's operator API, weights rotated over more
    than twice the 256 MB MALL for the bandwidth-bound cases: cfg1 (AWQ zero-point int4 g128,
    M=16, K=2560, N=9728), cfg4 (MoE E=128 top-8 H=2048 I=768, int4 g128 fp16 scales, T in
    {1,16,32,256,4096}) and cfg5 (MXFP4 E8M0 block-32 at K=8192,N=28672 and K=28672,N=8192, M in
    {1,16,4096}). Bytes and FLOPs count the algorithmic traffic (codes, scales, zero words,
    bf16 activations in and out; MoE: the distinct experts the route selected)."""
    import torch

    out = {}
    gen = torch.Generator(device=dev).manual_seed(11)
    # cfg1: AWQ dense decode
    M, K, N, g = 16, 2560, 9728, 128
    copies = []
    for _ in range(40):
        t = kernels.repack_w4(_rand_words((N, K // 8), gen, dev))
        sc = (torch.randn(K // g, N, generator=gen, device=dev).abs() * 0.02 + 1e-4).to(torch.float16)
        z = _rand_words((K // g, N // 8), gen, dev)
        copies.append((t, sc, z))
    x = make_x(M, K, 101, dev)
    us = _time_calls([lambda c=c: kernels.w4a8_linear(x, c[0], c[1], c[2], g) for c in copies], 80)
    nb = N * K // 2 + (K // g) * N * 2 + (K // g) * N // 2 + M * K * 2 + M * N * 2
    out["cfg1_awq_M16_K2560_N9728"] = _gbs(nb, us)
    del copies
    # cfg5: MXFP4
    for (K, N) in [(8192, 28672), (28672, 8192)]:
        copies = []
        for _ in range(5):
            t = kernels.repack_w4(_rand_words((N, K // 8), gen, dev), weight_is_e2m1=True)
            sc = torch.randint(119, 128, (K // 32, N), generator=gen, device=dev, dtype=torch.int32).to(torch.uint8)
            copies.append((t, sc))
        for M in (1, 16):
            x = make_x(M, K, 200 + M, dev)
            us = _time_calls([lambda c=c: kernels.w4a8_linear(x, c[0], c[1], None, 32, weight_is_e2m1=True)
                              for c in copies], 40)
            nb = N * K // 2 + (K // 32) * N + M * K * 2 + M * N * 2
            out[f"cfg5_mxfp4_M{M}_K{K}_N{N}"] = _gbs(nb, us)
        M = 4096
        x = make_x(M, K, 300, dev)
        q, s = kernels.act_quant(x)
        c = copies[0]
        us = _time_calls([lambda: kernels.w4a8_linear(x, c[0], c[1], None, 32, weight_is_e2m1=True, x_fp8=q,
                                                      act_scales=s)], 5)
        out[f"cfg5_mxfp4_M{M}_K{K}_N{N}"] = _tflops(2.0 * M * N * K, us)
        del copies
    # cfg4: MoE
    E, k, H, I, g = 128, 8, 2048, 768, 128
    layers = []
    for _ in range(2):
        w13 = kernels.repack_w4(_rand_words((E, 2 * I, H // 8), gen, dev))
        s13 = (torch.randn(E, H // g, 2 * I, generator=gen, device=dev).abs() * 0.02 + 1e-4).to(torch.float16)
        w2 = kernels.repack_w4(_rand_words((E, H, I // 8), gen, dev))
        s2 = (torch.randn(E, I // g, H, generator=gen, device=dev).abs() * 0.02 + 1e-4).to(torch.float16)
        layers.append((w13, s13, w2, s2))
    per_expert = 2 * I * H // 2 + (H // g) * 2 * I * 2 + H * I // 2 + (I // g) * H * 2
    for T in (1, 16, 32, 256, 4096):
        x = make_x(T, H, 400 + T, dev)
        logits = torch.randn(T, E, generator=gen, device=dev).to(torch.bfloat16)
        distinct = int(torch.topk(logits.float(), k, dim=-1).indices.unique().numel())
        calls = [lambda L=L: kernels.w4a8_moe(x, L[0], L[1], None, L[2], L[3], None, logits, k, True) for L in layers]
        us = _time_calls(calls, 20 if T < 4096 else 5)
        if T < 4096:
            r = _gbs(distinct * per_expert + 2 * T * H * 2, us)
        else:
            r = _tflops(2.0 * T * k * (H * 2 * I + I * H), us)
        r["distinct_experts"] = distinct
        out[f"cfg4_moe_T{T}"] = r
    del layers
    return out


def formats_leg(kernels, dev) -> dict:
    """The formats beyond the BASELINE configs, through the same operator API: the W4A16 arm
    (unquantized bf16 activations; GPTQ-sym int4 g128 at the gate_up shape K=4096, N=28672, M in
    {1, 16, 2048}) and NVFP4 (e2m1 + e4m3 block-16 scales + per-channel global; W4A8 at the cfg5
    gate_up shape K=8192, N=28672, M in {1, 16, 4096}, and W4A16 at M=1). Weights rotate over more
    than twice the MALL for the bandwidth-bound sizes; bytes count codes, scales (and the NVFP4
    global), bf16 activations in and out."""
    import torch

    out = {}
    gen = torch.Generator(device=dev).manual_seed(13)
    K, N, g = 4096, 28672, 128
    copies = []
    for _ in range(10):
        t = kernels.repack_w4(_rand_words((N, K // 8), gen, dev))
        sc = (torch.randn(K // g, N, generator=gen, device=dev).abs() * 0.02).to(torch.float16)
        copies.append((t, sc))
    for M in (1, 16):
        x = make_x(M, K, 600 + M, dev)
        us = _time_calls([lambda c=c: kernels.w4a16_linear(x, c[0], c[1], None, g, N) for c in copies], 40)
        out[f"w4a16_int4_M{M}_K{K}_N{N}"] = _gbs(algo_bytes(M, K, N), us)
    M = 2048
    x = make_x(M, K, 602, dev)
    c = copies[0]
    us = _time_calls([lambda: kernels.w4a16_linear(x, c[0], c[1], None, g, N)], 5)
    out[f"w4a16_int4_M{M}_K{K}_N{N}"] = _tflops(2.0 * M * N * K, us)
    del copies
    K, N = 8192, 28672
    copies = []
    for _ in range(5):
        t = kernels.repack_w4(_rand_words((N, K // 8), gen, dev), weight_is_e2m1=True)
        sc = (torch.rand(K // 16, N, generator=gen, device=dev) * 6 + 0.25).to(torch.float8_e4m3fn)
        gl = torch.rand(N, generator=gen, device=dev) * 1e-3 + 1e-4
        copies.append((t, sc, gl))
    nv_bytes = lambda M: N * K // 2 + (K // 16) * N + N * 4 + M * K * 2 + M * N * 2
    for M in (1, 16):
        x = make_x(M, K, 700 + M, dev)
        us = _time_calls([lambda c=c: kernels.w4a8_linear(x, c[0], c[1], c[2], 16, weight_is_e2m1=True)
                          for c in copies], 40)
        out[f"nvfp4_w4a8_M{M}_K{K}_N{N}"] = _gbs(nv_bytes(M), us)
    x = make_x(1, K, 701, dev)
    us = _time_calls([lambda c=c: kernels.w4a16_linear(x, c[0], c[1], c[2], 16, N, weight_is_e2m1=True)
                      for c in copies], 40)
    out[f"nvfp4_w4a16_M1_K{K}_N{N}"] = _gbs(nv_bytes(1), us)
    M = 4096
    x = make_x(M, K, 702, dev)
    q, s = kernels.act_quant(x)
    c = copies[0]
    us = _time_calls([lambda: kernels.w4a8_linear(x, c[0], c[1], c[2], 16, weight_is_e2m1=True, x_fp8=q,
                                                  act_scales=s)], 5)
    out[f"nvfp4_w4a8_M{M}_K{K}_N{N}"] = _tflops(2.0 * M * N * K, us)
    del copies
    return out


def producer_leg(kernels, dev, weights, steps: int = 100) -> dict:
    """The configs[1] sweep with its activations produced by the RMSNorm + residual-add producer, in
    two graph-replayed steps of 20 (norm, linear) pairs: `in_op_quant` runs rms_norm_add then
    w4a8_linear on bf16 x (the linear quantizes), `producer_pair` runs rms_norm_add_quant then
    w4a8_linear on the (x_fp8, act_scales) pair it emitted. Same weights as the headline step."""
    import torch

    norm = importlib.import_module("minisglang-rdna4_amd.layers.norm")
    gen = torch.Generator(device=dev).manual_seed(77)
    xs = [[make_x(M, K, 3000 + 10 * i + j, dev) for j, (K, N) in enumerate(SHAPES)] for i, M in enumerate(MS)]
    rs = [[make_x(M, K, 4000 + 10 * i + j, dev) for j, (K, N) in enumerate(SHAPES)] for i, M in enumerate(MS)]
    gains = {K: (torch.randn(K, generator=gen, device=dev) * 0.1 + 1.0).to(torch.bfloat16) for K, _ in SHAPES}

    def step(pair: bool):
        outs = []
        for i, M in enumerate(MS):
            for j, (K, N) in enumerate(SHAPES):
                t, sc = weights[i][j]
                if pair:
                    h, q, s = norm._rms_norm_add_quant(xs[i][j], rs[i][j], gains[K], 1e-6)
                    outs.append(kernels.w4a8_linear(h, t, sc, None, GROUP, x_fp8=q, act_scales=s))
                else:
                    h = norm._rms_norm_add(xs[i][j], rs[i][j], gains[K], 1e-6)
                    outs.append(kernels.w4a8_linear(h, t, sc, None, GROUP))
        return outs

    out = {}
    for name, pair in (("in_op_quant", False), ("producer_pair", True)):
        step(pair)
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step(pair)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            keep = step(pair)
        for _ in range(10):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            graph.replay()
        torch.cuda.synchronize()
        out[name] = {"us_per_step": round((time.perf_counter() - t0) * 1e6 / steps, 1)}
        del graph, keep
    aq = launches_per_step() - len(MS) * len(SHAPES)
    out["launches_per_step"] = {"in_op_quant": f"20 norms + {aq} act-quant + 20 GEMV",
                                "producer_pair": "20 norms (with the quant epilogue) + 20 GEMV"}
    return out


def launches_per_step() -> int:
    """Kernel launches of one configs[1] step (w4a8_linear_launch_count over its 20 calls)."""
    lib = importlib.import_module("minisglang-rdna4_amd._abi").load()
    return sum(lib.w4a8_linear_launch_count(M, N, K, 0, 0, 0, 0, GROUP, 0, 0) for M in MS for (K, N) in SHAPES)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--profile-kernel", action="store_true")
    ap.add_argument("--copy-calib", action="store_true")
    ap.add_argument("--read-floor", action="store_true",
                    help="time the streaming-read floor of one launch at the decode weight sizes and exit")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-configs", action="store_true")
    ap.add_argument("--profile-prefill", nargs=4, metavar=("FMT", "M", "K", "N"),
                    help="time one prefill GEMM (FMT int4, mxfp4 or nvfp4) and exit, for counter runs")
    ap.add_argument("--profile-moe", type=int, metavar="T",
                    help="time one configs[4] MoE call of T tokens and exit, for trace and counter runs")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one MI355X; --gpus {args.gpus} (WORLD_SIZE={world}) is not run. "
              f"Every GPU box of this build has one GPU; a figure at several GPUs is not measured.", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    kernels = importlib.import_module("minisglang-rdna4_amd.quant.kernels")

    if args.copy_calib:
        n = 256 << 20
        a = torch.empty(n, dtype=torch.uint8, device=dev)
        b = torch.empty(n, dtype=torch.uint8, device=dev)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes_read": n, "copy_calib_bytes_written": n}))
        return 0
    if args.read_floor:
        print(json.dumps({"read_floor": read_floor(dev)}))
        return 0
    if args.profile_kernel:
        r = roofline_leg(kernels, dev)
        print(json.dumps(r))
        return 0
    if args.profile_moe:
        print(json.dumps(profile_moe(kernels, dev, args.profile_moe)))
        return 0
    if args.profile_prefill:
        f, m, k, n = args.profile_prefill
        print(json.dumps(profile_prefill(kernels, dev, f, int(m), int(k), int(n))))
        return 0

    # ---- sweep setup: 5 weight copies (one per M), activations per (M, shape)
    gen = torch.Generator(device=dev).manual_seed(1234)
    weights = [[make_weights(kernels, K, N, gen, dev) for (K, N) in SHAPES] for _ in MS]
    xs = [[make_x(M, K, 1000 + 10 * i + j, dev) for j, (K, N) in enumerate(SHAPES)] for i, M in enumerate(MS)]
    step_bytes = sum(algo_bytes(M, K, N) for M in MS for (K, N) in SHAPES)
    weight_bytes = sum(t.numel() + s.numel() * 2 for row in weights for (t, s) in row)

    def step():
        outs = []
        for i, M in enumerate(MS):
            for j, (K, N) in enumerate(SHAPES):
                t, s = weights[i][j]
                outs.append(kernels.w4a8_linear(xs[i][j], t, s, None, GROUP))
        return outs

    # eager warm-up, then capture one step
    step()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        graph_outs = step()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    del graph_outs
    ms_per_step = elapsed * 1e3 / args.steps
    value = step_bytes * args.steps / elapsed / 1e9

    # per-shape GEMV-only view (events around graph replays of one call each would add a graph per
    # shape; the roofline leg covers the dominant shape)
    roof = roofline_leg(kernels, dev)
    per_shape = decode_shapes_leg(kernels, dev)
    prefill = None if args.no_prefill else prefill_leg(kernels, dev)
    others = None if args.no_configs else configs_leg(kernels, dev)
    producer = None if args.no_configs else producer_leg(kernels, dev, weights)
    formats = None if args.no_configs else formats_leg(kernels, dev)
    cpu = None if args.no_cpu_baseline else cpu_baseline_leg()

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 x int4, f32 accumulate",
        "data": "synthetic (seeded): GPTQ-sym int4 g128 codes U{0..15}, fp16 scales |N(0,0.02)|, bf16 N(0,1) "
                "activations with 0.1% channels x50",
        "config": {
            "workload": "configs[1]: decode W4A8 GEMM sweep at Llama-3-8B layer shapes, M in {1,2,4,8,16}; one step = "
                        "20 calls (per-token act quant + GEMM each), HIP-graph replayed",
            "launches_per_step": launches_per_step(),
            "shapes_KxN": [f"{K}x{N}" for K, N in SHAPES],
            "M": MS,
            "group_size": GROUP,
            "algorithmic_bytes_per_step": step_bytes,
            "weight_bytes_cycled": weight_bytes,
            "frac_of_hbm_peak_whole_step": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        "decode_per_shape": per_shape,
        "prefill_config3": prefill,
        "other_configs": others,
        "next_formats": formats,
        "producer_norm_step": producer,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
