"""MXFP4 (OCP E2M1 codes + E8M0 per-32-block exponents) load-time conversion.

Same names and contracts as python/minisgl/quant/mxfp4.py of the reference: the e2m1 nibbles are
repacked verbatim into the (N, K/8) int32 op container (code j of a word at bits 4j..4j+3, low
nibble of each checkpoint byte = even K), and the E8M0 byte is passed through untouched -- the
MI355X kernels feed it straight to the scaled f8f6f4 MFMA as the B block scale.
"""
from __future__ import annotations

import torch

# OCP E2M1 codebook by raw code (bit3 sign, bits2-1 exponent, bit0 mantissa); mxfp4.py:37-38.
FP4_E2M1_LUT = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]

OCP_MX_BLOCK_SIZE = 32
E8M0_BIAS = 127


def unpack_e2m1_nibbles(weight_packed: torch.Tensor) -> torch.Tensor:
    """(N, K//2) uint8 -> (N, K) uint8 codes; low nibble = lower (even) K index (mxfp4.py:44-52)."""
    assert weight_packed.dtype == torch.uint8 and weight_packed.dim() == 2, (weight_packed.dtype, weight_packed.shape)
    lo = weight_packed & 0x0F
    hi = (weight_packed >> 4) & 0x0F
    return torch.stack([lo, hi], dim=-1).reshape(weight_packed.shape[0], weight_packed.shape[1] * 2)


def pack_codes_to_int32(codes: torch.Tensor) -> torch.Tensor:
    """(N, K) codes -> (N, K//8) int32, code j at bits [4j, 4j+3] (mxfp4.py:55-69)."""
    n, k = codes.shape
    assert k % 8 == 0, f"K={k} must be a multiple of 8 for int32 packing"
    c = (codes.to(torch.int64) & 0xF).reshape(n, k // 8, 8)
    sh = torch.arange(0, 32, 4, dtype=torch.int64, device=codes.device)
    words = (c << sh).sum(-1)
    return (words & 0xFFFFFFFF).to(torch.int32)


# E8M0 codes whose power of two 2^(code-127) falls outside fp16's normal range (2^-14 .. 2^15):
# below code 113 (code 0 excluded: it is the 2^-127 "zero" code, counted on its own) or above 142
_E8M0_FP16_LO, _E8M0_FP16_HI = E8M0_BIAS - 14, E8M0_BIAS + 15


def e8m0_scale_health(weight_scale: torch.Tensor) -> dict:
    """Load-time report on an E8M0 scale tensor (the contract of python/minisgl/quant/mxfp4.py:115-131):
    the unbiased exponent window, the blocks carrying the NaN code (255) or the zero code (0), and
    the blocks whose scale an fp16 path could not hold. One 256-bin histogram of the codes gives
    every figure."""
    if weight_scale.dtype != torch.uint8:
        raise TypeError(f"E8M0 scales must be uint8 codes, got {weight_scale.dtype}")
    if weight_scale.numel() == 0:
        raise ValueError("E8M0 scale tensor is empty")
    hist = torch.bincount(weight_scale.reshape(-1).to(torch.int64), minlength=256).cpu()
    present = torch.nonzero(hist).flatten()
    return {
        "exp_min": int(present[0]) - E8M0_BIAS,
        "exp_max": int(present[-1]) - E8M0_BIAS,
        "e8m0_nan_groups": int(hist[0xFF]),
        "e8m0_zero_code_groups": int(hist[0]),
        "would_saturate_fp16": int(hist[1:_E8M0_FP16_LO].sum() + hist[_E8M0_FP16_HI + 1:].sum()),
    }


def _as_op_words(weight_packed: torch.Tensor) -> torch.Tensor:
    """Checkpoint e2m1 bytes (..., K//2) uint8 (low nibble = even K) as the op container (..., K//8)
    int32 (code j of a word at bits 4j..4j+3). That container is the bytes themselves read as
    little-endian words: byte b of a word holds codes 2b (low nibble) and 2b + 1, i.e. code i at
    bits 4i, so the conversion is a copy into a word view, with no per-code arithmetic."""
    if weight_packed.dtype != torch.uint8:
        raise TypeError(f"e2m1 codes must be uint8 bytes, got {weight_packed.dtype}")
    if weight_packed.shape[-1] % 4:
        raise ValueError(f"K={weight_packed.shape[-1] * 2} must be a multiple of 8 for int32 words")
    return weight_packed.contiguous().view(torch.int32).clone()


def _check_mx_pair(weight_packed: torch.Tensor, weight_scale: torch.Tensor, nd: int) -> tuple:
    if weight_packed.dim() != nd or weight_scale.dim() != nd:
        raise ValueError(f"expected {nd}-D weight and scale, got {tuple(weight_packed.shape)} and "
                         f"{tuple(weight_scale.shape)}")
    k = weight_packed.shape[-1] * 2
    if tuple(weight_scale.shape[:-1]) != tuple(weight_packed.shape[:-1]):
        raise ValueError(f"weight rows {tuple(weight_packed.shape[:-1])} and scale rows "
                         f"{tuple(weight_scale.shape[:-1])} differ")
    if weight_scale.shape[-1] * OCP_MX_BLOCK_SIZE != k:
        raise ValueError(f"{weight_scale.shape[-1]} scale blocks for K={k} (expected K/{OCP_MX_BLOCK_SIZE})")
    return (*weight_packed.shape[:-1], k)


def _mx_result(weight_packed: torch.Tensor, weight_scale: torch.Tensor, shape: tuple) -> dict:
    return {
        "w_packed": _as_op_words(weight_packed),
        "scales": weight_scale.contiguous(),  # E8M0 bytes verbatim: the scaled MFMA's B block scale
        "w_zeros": None,
        "group_size": OCP_MX_BLOCK_SIZE,
        "scale_info": e8m0_scale_health(weight_scale),
        "shape": shape,
    }


def convert_mxfp4_weight(weight_packed: torch.Tensor, weight_scale: torch.Tensor) -> dict:
    """One MXFP4 matrix (contract of python/minisgl/quant/mxfp4.py:168-206): (N, K//2) uint8 codes
    and (N, K//32) uint8 E8M0 -> w_packed (N, K//8) int32, scales verbatim, w_zeros None,
    group_size 32, scale_info, shape (N, K)."""
    return _mx_result(weight_packed, weight_scale, _check_mx_pair(weight_packed, weight_scale, 2))


def convert_mxfp4_moe_e8m0(weight_packed: torch.Tensor, weight_scale: torch.Tensor) -> dict:
    """Stacked experts (contract of python/minisgl/quant/mxfp4.py:134-165): (E, N, K//2) and
    (E, N, K//32) -> w_packed (E, N, K//8) int32, scales verbatim, scale_is_e8m0 True, and the
    rest as for one matrix. The word view converts every expert at once with no transient beyond
    the output."""
    out = _mx_result(weight_packed, weight_scale, _check_mx_pair(weight_packed, weight_scale, 3))
    out["scale_is_e8m0"] = True
    return out


def dequant_reference(weight_packed: torch.Tensor, weight_scale: torch.Tensor) -> torch.Tensor:
    """E2M1(code) * 2^(s-127) as (N, K) float32 (mxfp4.py:262-275)."""
    codes = unpack_e2m1_nibbles(weight_packed).to(torch.int64)
    lut = torch.tensor(FP4_E2M1_LUT, dtype=torch.float32, device=weight_packed.device)
    w = lut[codes]
    scale = torch.pow(torch.tensor(2.0, device=weight_packed.device), weight_scale.to(torch.int32).float() - E8M0_BIAS)
    return w * scale.repeat_interleave(OCP_MX_BLOCK_SIZE, dim=-1)
