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


def e8m0_scale_health(weight_scale: torch.Tensor) -> dict:
    """Counts of the special E8M0 codes (0 -> 2^-127, 255 -> NaN/+inf) and the exponent window
    (mxfp4.py:115-131)."""
    assert weight_scale.dtype == torch.uint8, weight_scale.dtype
    exp = weight_scale.to(torch.int32) - E8M0_BIAS
    return {
        "exp_min": int(exp.min()), "exp_max": int(exp.max()),
        "e8m0_nan_groups": int((weight_scale == 0xFF).sum()),
        "e8m0_zero_code_groups": int((weight_scale == 0).sum()),
        "would_saturate_fp16": int(((exp > 15) | ((exp < -14) & (weight_scale != 0))).sum()),
    }


def convert_mxfp4_weight(weight_packed: torch.Tensor, weight_scale: torch.Tensor) -> dict:
    """One MXFP4 matrix: (N, K//2) uint8 + (N, K//32) uint8 -> {w_packed (N, K//8) int32,
    scales (N, K//32) uint8 E8M0 (verbatim), w_zeros None, group_size 32, scale_info}
    (mxfp4.py:168-206)."""
    n, k_half = weight_packed.shape
    k = k_half * 2
    ns, k_groups = weight_scale.shape
    assert ns == n, f"row mismatch: weight {n} vs scale {ns}"
    assert k_groups == k // OCP_MX_BLOCK_SIZE, f"scale groups {k_groups} != K//32 = {k // OCP_MX_BLOCK_SIZE}"
    return {
        "w_packed": pack_codes_to_int32(unpack_e2m1_nibbles(weight_packed)),
        "scales": weight_scale.contiguous(),
        "w_zeros": None,
        "group_size": OCP_MX_BLOCK_SIZE,
        "scale_info": e8m0_scale_health(weight_scale),
        "shape": (n, k),
    }


def convert_mxfp4_moe_e8m0(weight_packed: torch.Tensor, weight_scale: torch.Tensor) -> dict:
    """Stacked experts: (E, N, K//2) + (E, N, K//32) -> {w_packed (E, N, K//8) int32, scales
    (E, N, K//32) uint8 verbatim, ...} (mxfp4.py:134-165). Converted per expert so the int64
    nibble transient stays one matrix in size."""
    assert weight_packed.dim() == 3 and weight_scale.dim() == 3, (weight_packed.shape, weight_scale.shape)
    e, n, k_half = weight_packed.shape
    k = k_half * 2
    es, ns, k_groups = weight_scale.shape
    assert (es, ns) == (e, n), f"shape mismatch: weight {(e, n)} vs scale {(es, ns)}"
    assert k_groups == k // OCP_MX_BLOCK_SIZE, f"scale groups {k_groups} != K//32 = {k // OCP_MX_BLOCK_SIZE}"
    w_out = torch.empty((e, n, k // 8), dtype=torch.int32, device=weight_packed.device)
    for i in range(e):
        w_out[i] = pack_codes_to_int32(unpack_e2m1_nibbles(weight_packed[i]))
    return {
        "w_packed": w_out,
        "scales": weight_scale.contiguous(),
        "w_zeros": None,
        "group_size": OCP_MX_BLOCK_SIZE,
        "scale_is_e8m0": True,
        "scale_info": e8m0_scale_health(weight_scale),
        "shape": (e, n, k),
    }


def dequant_reference(weight_packed: torch.Tensor, weight_scale: torch.Tensor) -> torch.Tensor:
    """E2M1(code) * 2^(s-127) as (N, K) float32 (mxfp4.py:262-275)."""
    codes = unpack_e2m1_nibbles(weight_packed).to(torch.int64)
    lut = torch.tensor(FP4_E2M1_LUT, dtype=torch.float32, device=weight_packed.device)
    w = lut[codes]
    scale = torch.pow(torch.tensor(2.0, device=weight_packed.device), weight_scale.to(torch.int32).float() - E8M0_BIAS)
    return w * scale.repeat_interleave(OCP_MX_BLOCK_SIZE, dim=-1)
