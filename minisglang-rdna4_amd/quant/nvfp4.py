"""NVFP4 (compressed-tensors `nvfp4-pack-quantized`, modelopt NVFP4) load-time conversion.

Same names and contracts as python/minisgl/quant/nvfp4.py of the reference. NVFP4 shares MXFP4's
E2M1 codes and differs in the scale: an e4m3 block scale per 16 elements times a per-tensor f32
global. Both levels are kept (the reference's "split" form, exact; the fp16 "fold" is lossy): the
e4m3 bytes pass through verbatim and the global becomes a per-OUTPUT-CHANNEL f32 multiplier vector,
so the gate|up concat and the per-expert stack carry it as ordinary tensors. The kernels take the
vector in the zeros slot (its f32 bits viewed as int32) and multiply each group's partial sum by
e4m3(block) * global.

The two producers spell the global reciprocally: compressed-tensors `weight_global_scale` is a
divisor (448*6/amax), modelopt `weight_scale_2` a multiplier (amax/(448*6)). The caller names the
checkpoint field it read and the direction follows from that name alone
(nvfp4.py:70-130 of the reference).
"""
from __future__ import annotations

import torch

from .mxfp4 import FP4_E2M1_LUT, pack_codes_to_int32, unpack_e2m1_nibbles

NVFP4_GROUP_SIZE = 16

# checkpoint field -> whether the stored global is the reciprocal of the multiplier
NVFP4_GLOBAL_SCALE_IS_RECIPROCAL = {
    "weight_global_scale": True,  # compressed-tensors: divide
    "weight_scale_2": False,  # modelopt: multiply
}


def _global_is_reciprocal(global_field: str) -> bool:
    try:
        return NVFP4_GLOBAL_SCALE_IS_RECIPROCAL[global_field]
    except KeyError:
        raise ValueError(
            f"unknown NVFP4 global-scale field {global_field!r}: the global is a divisor in compressed-tensors "
            f"('weight_global_scale') and a multiplier in modelopt ('weight_scale_2'); add the new spelling to "
            f"NVFP4_GLOBAL_SCALE_IS_RECIPROCAL with its direction") from None


def nvfp4_global_multiplier(global_scale: torch.Tensor, *, global_field: str) -> torch.Tensor:
    """The per-tensor global as a direction-normalised 0-dim f32 MULTIPLIER (nvfp4.py:103-131):
    the kernels only multiply. Non-finite or non-positive values are refused."""
    reciprocal = _global_is_reciprocal(global_field)
    g = global_scale.to(torch.float32).reshape(())
    if not bool(torch.isfinite(g)) or float(g) <= 0.0:
        raise ValueError(f"NVFP4 global scale for field {global_field!r} is {float(g)!r}; it must be finite and > 0")
    mul = (1.0 / g) if reciprocal else g
    if not bool(torch.isfinite(mul)) or float(mul) <= 0.0:
        raise ValueError(f"NVFP4 global scale for field {global_field!r} normalised to {float(mul)!r}")
    return mul


def split_nvfp4_scale(weight_scale: torch.Tensor, global_scale: torch.Tensor, *, global_field: str,
                      out_features: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(N, K//16) e4m3 block scale + per-tensor global -> (the block scale byte-verbatim as
    float8_e4m3fn, the (N,) f32 global multiplier) (nvfp4.py:134-179). uint8 block scales are
    bitcast, never value-converted."""
    if weight_scale.ndim != 2:
        raise ValueError(f"NVFP4 leaf block scale must be (N, K//{NVFP4_GROUP_SIZE}); got {tuple(weight_scale.shape)}")
    mul = nvfp4_global_multiplier(global_scale, global_field=global_field)
    if weight_scale.dtype == torch.uint8:
        block = weight_scale.view(torch.float8_e4m3fn)
    elif weight_scale.dtype == torch.float8_e4m3fn:
        block = weight_scale
    else:
        raise ValueError(f"NVFP4 block scale must be float8_e4m3fn (or its raw uint8 bytes); got {weight_scale.dtype}")
    n = int(weight_scale.shape[0]) if out_features is None else int(out_features)
    return block.contiguous(), torch.full((n,), float(mul), dtype=torch.float32, device=weight_scale.device)


def _block_scale(weight_scale: torch.Tensor) -> torch.Tensor:
    if weight_scale.dtype == torch.uint8:
        return weight_scale.view(torch.float8_e4m3fn)
    if weight_scale.dtype == torch.float8_e4m3fn:
        return weight_scale
    raise ValueError(f"NVFP4 scale must be float8_e4m3fn or its uint8 bytes (the two-level form); got "
                     f"{weight_scale.dtype}. fp16 here would be the lossy fold, which this build does not load")


def convert_nvfp4_weight(weight_packed: torch.Tensor, weight_scale: torch.Tensor) -> dict:
    """One NVFP4 matrix -> the e2m1 op layout (nvfp4.py:323-347): weight_packed (N, K//2) uint8
    nibbles -> w_packed (N, K//8) int32 codes verbatim; weight_scale (N, K//16) e4m3 passes through."""
    n, k_half = weight_packed.shape
    k = k_half * 2
    if tuple(weight_scale.shape) != (n, k // NVFP4_GROUP_SIZE):
        raise ValueError(f"NVFP4 scale must be (N, K//16)=({n}, {k // NVFP4_GROUP_SIZE}); got {tuple(weight_scale.shape)}")
    return {
        "w_packed": pack_codes_to_int32(unpack_e2m1_nibbles(weight_packed)),
        "scales": _block_scale(weight_scale).contiguous(),
        "group_size": NVFP4_GROUP_SIZE,
        "shape": (n, k),
    }


def convert_nvfp4_moe(weight_packed: torch.Tensor, weight_scale: torch.Tensor) -> dict:
    """Stacked experts (nvfp4.py:350-371): (E, N, K//2) uint8 + (E, N, K//16) e4m3 ->
    {w_packed (E, N, K//8) int32, scales (E, N, K//16) e4m3, group_size 16}, one expert at a time."""
    assert weight_packed.ndim == 3 and weight_scale.ndim == 3, (weight_packed.shape, weight_scale.shape)
    e, n, k_half = weight_packed.shape
    k = k_half * 2
    w_out = torch.empty((e, n, k // 8), dtype=torch.int32, device=weight_packed.device)
    s_out = torch.empty((e, n, k // NVFP4_GROUP_SIZE), dtype=torch.float8_e4m3fn, device=weight_packed.device)
    for i in range(e):
        conv = convert_nvfp4_weight(weight_packed[i], weight_scale[i])
        w_out[i] = conv["w_packed"]
        s_out[i] = conv["scales"]
    return {"w_packed": w_out, "scales": s_out, "group_size": NVFP4_GROUP_SIZE, "shape": (e, n, k)}


def dequant_reference(weight_packed: torch.Tensor, weight_scale: torch.Tensor,
                      weight_global: torch.Tensor) -> torch.Tensor:
    """f32 dense weight (N, K) = e2m1(code) * e4m3(block scale) * global[n] (nvfp4.py:374-421,
    two-level form), for checks on the host."""
    codes = unpack_e2m1_nibbles(weight_packed).to(torch.int64)
    lut = torch.tensor(FP4_E2M1_LUT, dtype=torch.float32, device=weight_packed.device)
    vals = lut[codes]
    s = _block_scale(weight_scale).to(torch.float32).repeat_interleave(NVFP4_GROUP_SIZE, dim=1)
    return vals * s * weight_global.to(torch.float32).reshape(-1, 1)
