"""CPU baseline for bench.py -- TEST INFRASTRUCTURE ONLY (the cpu_baseline leg).

Restates the reference's CPU dequantize-then-matmul path for W4A8 (tools/moe_parity.py:23-43,
tools/qwen3_5_moe_awq_convert_test.py:40-69, python/minisgl/quant/mxfp4.py:262-275): quantize x per
token to e4m3 and back to f32, dequantize W = scale * (q - zero) to an f32 (N, K) matrix, then an
f32 matmul. torch on the CPU, all host cores.
"""
from __future__ import annotations

import os
import time

import torch


def _e4m3_roundtrip(x: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    amax = xf.abs().amax(dim=1, keepdim=True)
    s = (amax / 448.0).clamp_min(1e-8)
    q = (xf * (1.0 / s)).to(torch.float8_e4m3fn)
    return q.float() * s


def _dequant_int4(w_packed: torch.Tensor, scales: torch.Tensor, group: int) -> torch.Tensor:
    N, K8 = w_packed.shape
    sh = torch.arange(0, 32, 4, dtype=torch.int32)
    q = ((w_packed.unsqueeze(-1) >> sh) & 15).reshape(N, K8 * 8).float()
    return (q - 8.0) * scales.float().t().repeat_interleave(group, dim=1)


def cpu_model() -> str:
    """The host CPU as lscpu reports it: 'Model name', with the family / model / stepping numbers
    and the socket count (a virtualized host may report only a family name such as "AMD EPYC");
    /proc/cpuinfo's model name if lscpu is missing."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        f = {k.strip(): v.strip() for k, v in (ln.split(":", 1) for ln in out.splitlines() if ":" in ln)}
        if f.get("Model name"):
            extra = ", ".join(f"{k.lower()} {f[k]}" for k in ("CPU family", "Model", "Stepping", "Socket(s)") if k in f)
            return f"{f['Model name']} ({extra})" if extra else f["Model name"]
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def run(shapes, Ms, group: int, seed: int = 0, repeats: int = 5) -> dict:
    """Times the reference CPU path for every (K, N) shape at every M (one call = act round trip +
    dequant + matmul, as each reference CPU call dequantizes), `repeats` times over the whole set;
    returns bytes per pass, the median pass time (seconds, dequant_s, matmul_s taken from that
    pass), every pass's total, cores and the CPU model."""
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(seed)
    weights = []
    for K, N in shapes:
        codes = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int32)
        w = ((codes.reshape(N, K // 8, 8) << torch.arange(0, 32, 4, dtype=torch.int32)).sum(-1)).to(torch.int32)
        s = (torch.randn(K // group, N, generator=g).abs() * 0.02).to(torch.float16)
        xs = [torch.randn(M, K, generator=g).to(torch.bfloat16) for M in Ms]
        weights.append((K, N, w, s, xs))
        del codes
    passes = []
    for _ in range(repeats):
        t_deq = t_mm = 0.0
        nbytes = 0
        for K, N, w, s, xs in weights:
            for M, x in zip(Ms, xs):
                t0 = time.perf_counter()
                xd = _e4m3_roundtrip(x)
                wd = _dequant_int4(w, s, group)
                t1 = time.perf_counter()
                y = (xd @ wd.t()).to(torch.bfloat16)
                t2 = time.perf_counter()
                t_deq += t1 - t0
                t_mm += t2 - t1
                nbytes += N * K // 2 + (K // group) * N * 2 + M * K * 2 + M * N * 2
                del y, wd
        passes.append((t_deq + t_mm, t_deq, t_mm, nbytes))
    passes.sort()
    tot, deq, mm, nbytes = passes[len(passes) // 2]
    return {"bytes": nbytes, "seconds": tot, "dequant_s": deq, "matmul_s": mm, "cores": cores,
            "repeats": repeats, "all_seconds": [round(p[0], 4) for p in passes], "cpu_model": cpu_model()}
