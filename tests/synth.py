"""Seeded synthetic inputs for the five BASELINE workloads (shared by tests and bench.py).

Everything is generated on the CPU with a torch.Generator, so the same seed yields the same
bytes on every machine; callers move tensors to the GPU themselves.
"""
from __future__ import annotations

import torch

E8M0_LO, E8M0_HI = 127 - 8, 127  # exponents uniform in [-8, 0]


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def activations(M: int, K: int, seed: int, outliers: bool = False, dtype=torch.bfloat16) -> torch.Tensor:
    """bf16 N(0,1); with outliers, 0.1% of channels (a fixed index set per seed) scaled by 50."""
    g = gen(seed)
    x = torch.randn(M, K, generator=g)
    if outliers:
        n_out = max(1, K // 1000)
        idx = torch.randperm(K, generator=gen(seed + 7))[:n_out]
        x[:, idx] *= 50.0
    return x.to(dtype)


def pack_rows(codes: torch.Tensor) -> torch.Tensor:
    """(..., K) codes 0..15 -> (..., K/8) int32, nibble j of word i = code 8i+j (op layout)."""
    *lead, K = codes.shape
    c = codes.to(torch.int64).reshape(*lead, K // 8, 8)
    sh = torch.arange(0, 32, 4, dtype=torch.int64)
    w = (c << sh).sum(-1)
    return (w & 0xFFFFFFFF).to(torch.int32)


def int4_weight(N: int, K: int, group: int, seed: int, asym: bool, scale_floor: float = 0.0, E: int | None = None):
    """Op-layout int4 weight: codes U{0..15}; fp16 scales |N(0,0.02)| (+floor); zeros U{0..15}
    packed 8 channels per int32 along N when asym, else None (zero point 8).
    Shapes: w (N, K/8) / scales (K/g, N) / zeros (K/g, N/8), or with a leading E."""
    g = gen(seed)
    lead = () if E is None else (E,)
    codes = torch.randint(0, 16, (*lead, N, K), generator=g, dtype=torch.int32)
    scales = (torch.randn(*lead, K // group, N, generator=g).abs() * 0.02 + scale_floor).to(torch.float16)
    zeros = None
    if asym:
        z = torch.randint(0, 16, (*lead, K // group, N), generator=g, dtype=torch.int32)
        zeros = pack_rows(z)
    return pack_rows(codes), scales, zeros


def mxfp4_weight(N: int, K: int, seed: int, E: int | None = None):
    """MXFP4: e2m1 codes uniform over the 16 values, E8M0 block-32 scales with exponents in [-8, 0]
    as group-major (K/32, N) uint8."""
    g = gen(seed)
    lead = () if E is None else (E,)
    codes = torch.randint(0, 16, (*lead, N, K), generator=g, dtype=torch.int32)
    scales = torch.randint(E8M0_LO, E8M0_HI + 1, (*lead, K // 32, N), generator=g, dtype=torch.int32).to(torch.uint8)
    return pack_rows(codes), scales


def nvfp4_weight(N: int, K: int, seed: int, E: int | None = None):
    """NVFP4 (python/minisgl/quant/nvfp4.py:1-60): e2m1 codes uniform over the 16 values; e4m3
    block-16 scales as group-major (K/16, N) float8_e4m3fn, positive, |N(0,1)| * 8 + 0.5 (so they
    span several binades and use the mantissa bits); a per-output-channel f32 global multiplier
    |N(0, 1e-3)| + 1e-4 (the modelopt spelling, already direction-normalised)."""
    g = gen(seed)
    lead = () if E is None else (E,)
    codes = torch.randint(0, 16, (*lead, N, K), generator=g, dtype=torch.int32)
    scales = (torch.randn(*lead, K // 16, N, generator=g).abs() * 8 + 0.5).to(torch.float8_e4m3fn)
    glob = torch.randn(*lead, N, generator=g).abs() * 1e-3 + 1e-4
    return pack_rows(codes), scales, glob.to(torch.float32)


def router_logits(T: int, E: int, seed: int, dtype=torch.bfloat16) -> torch.Tensor:
    return torch.randn(T, E, generator=gen(seed)).to(dtype)


def bits16(t: torch.Tensor):
    """bf16/fp16 tensor -> numpy uint16 bit patterns."""
    return t.contiguous().view(torch.int16).numpy().view("uint16")
