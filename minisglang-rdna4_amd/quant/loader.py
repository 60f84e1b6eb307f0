"""Checkpoint ingestion for the W4A8 path: safetensors tensors into the methods' declared buffers.

The reference's loader (python/minisgl/models/weight.py with layers/base.py:122-171 and
quant/method.py:402-445) reads each module's checkpoint tensors by name into the buffers its
quant method declared in create_weights, checks them (a quantized dtype mismatch is an error, not a
cast), merges fused projections (gate|up, q|k|v) along the output axis, stacks routed experts, and
then runs process_weights_after_load / post_load. This module does the same for one linear or one
MoE block at a time, driven by QuantConfig.for_module, so a model's loader only has to name its
modules:

    tensors = read_safetensors(["model-00001-of-00002.safetensors", ...])
    method, layer = build_linear(quant, "model.layers.0.mlp.gate_up_proj", hidden, 2 * inter, tensors,
                                 parts=["model.layers.0.mlp.gate_proj", "model.layers.0.mlp.up_proj"])
    y = method.apply(layer, x, None)

NVFP4's per-tensor global arrives under its producer's field name (compressed-tensors
`weight_global_scale`, a divisor; modelopt `weight_scale_2`, a multiplier) and is normalised by
quant.nvfp4.split_nvfp4_scale into the per-output-channel vector the method declares as
`weight_global`. modelopt and AMD Quark name the packed 4-bit codes `weight` (uint8) where
compressed-tensors says `weight_packed`; the loader reads either (python/minisgl/models/weight.py:
1025-1045, which renames on the uint8 dtype the same way). Activation calibration tensors
(`input_global_scale`, `input_scale`) and compressed-tensors' `weight_shape` are not used.
"""
from __future__ import annotations

import importlib
from types import SimpleNamespace
from typing import Iterable

import torch

from . import method as _method
from . import nvfp4 as _nvfp4
from .config import QuantConfig

_pkg = __name__.rsplit(".", 2)[0]

_QUANT_DTYPES = (torch.int32, torch.uint8, torch.float8_e4m3fn, torch.int8)


def read_safetensors(paths: Iterable[str], device: str | torch.device = "cpu") -> dict[str, torch.Tensor]:
    """All tensors of the given .safetensors files, by name (a later file wins a duplicate name)."""
    from safetensors.torch import load_file

    out: dict[str, torch.Tensor] = {}
    for p in paths:
        out.update(load_file(str(p), device=str(device)))
    return out


def _coerce(name: str, declared: torch.Tensor, got: torch.Tensor) -> torch.Tensor:
    """The checkpoint tensor in the declared buffer's shape and dtype. Shapes must match exactly.
    Quantized payloads keep their bits: uint8 and float8_e4m3fn are the same bytes (a bitcast),
    any other quantized mismatch is refused; floating-point scales are value-converted."""
    if tuple(got.shape) != tuple(declared.shape):
        raise ValueError(f"{name}: checkpoint shape {tuple(got.shape)} != declared {tuple(declared.shape)}")
    if got.dtype == declared.dtype:
        return got
    if {got.dtype, declared.dtype} == {torch.uint8, torch.float8_e4m3fn}:
        return got.view(declared.dtype)
    if got.dtype in _QUANT_DTYPES or declared.dtype in _QUANT_DTYPES:
        raise TypeError(f"{name}: weight dtype mismatch, model {declared.dtype} vs checkpoint {got.dtype}")
    return got.to(declared.dtype)


def _nvfp4_global(tensors: dict, prefix: str) -> torch.Tensor:
    """The module's per-tensor global as its (N,) f32 multiplier vector, N = the module's rows."""
    w = tensors.get(f"{prefix}.weight_packed", tensors.get(f"{prefix}.weight"))
    if w is None:
        raise KeyError(f"missing checkpoint tensor {prefix}.weight_packed")
    n = int(w.shape[0])
    for field in ("weight_global_scale", "weight_scale_2"):
        key = f"{prefix}.{field}"
        if key in tensors:
            mul = _nvfp4.nvfp4_global_multiplier(tensors[key], global_field=field)
            return torch.full((n,), float(mul), dtype=torch.float32)
    raise KeyError(f"{prefix}: NVFP4 needs a per-tensor global ('weight_global_scale' or 'weight_scale_2')")


def _fetch(tensors: dict, prefix: str, attr: str, declared: torch.Tensor, nvfp4: bool) -> torch.Tensor:
    if nvfp4 and attr == "weight_global":
        return _nvfp4_global(tensors, prefix)
    key = f"{prefix}.{attr}"
    alt = f"{prefix}.weight"
    if key not in tensors and attr == "weight_packed" and alt in tensors and tensors[alt].dtype == torch.uint8:
        key = alt  # modelopt / Quark name the packed codes `weight`; a full-precision weight is never uint8
    if key not in tensors:
        raise KeyError(f"missing checkpoint tensor {key}")
    return tensors[key]


# output-axis of each declared buffer (the axis fused projections concatenate along); None: shared
def _n_axis(quant: QuantConfig | None, attr: str) -> int | None:
    if quant is None:
        return 0  # unquantized weight (N, K)
    if attr == "g_idx":
        return None
    if quant.is_compressed_tensors:
        return 0  # weight_packed (N, K/8 | K/2), weight_scale (N, K/g), weight_zero_point (N/8, K/g), weight_global (N,)
    return 1  # AWQ qweight (K, N/8), GPTQ qweight (K/8, N); scales (K/g, N); qzeros (K/g, N/8)


def _declared(layer) -> dict[str, torch.Tensor]:
    return {k: v for k, v in vars(layer).items() if isinstance(v, torch.Tensor) and not k.startswith("_")}


def build_linear(quant: QuantConfig | None, name: str, in_features: int, out_features: int,
                 tensors: dict[str, torch.Tensor], *, parts: list[str] | None = None,
                 device: str | torch.device = "cuda"):
    """(method, layer) of linear module `name` loaded from `tensors`. `parts`: the checkpoint
    prefixes of a fused projection (e.g. gate_proj and up_proj of a gate_up layer), concatenated
    along the output axis in order; their output widths must sum to out_features."""
    q = quant.for_module(name) if quant is not None else None
    m = _method.create_linear_method(q)
    layer = SimpleNamespace()
    m.create_weights(layer, out_features, in_features)
    decl = _declared(layer)
    nvfp4 = q is not None and q.is_nvfp4
    for attr, buf in decl.items():
        prefixes = parts or [name]
        pieces = [_fetch(tensors, p, attr, buf, nvfp4) for p in prefixes]
        ax = _n_axis(q, attr)
        if len(pieces) == 1 or ax is None:
            got = pieces[0]
        else:
            dts = {t.dtype for t in pieces}
            if len(dts) != 1:
                raise TypeError(f"{name}.{attr}: fused parts disagree on dtype {dts}")
            got = torch.cat(pieces, dim=ax)
        if q is None:
            # an unquantized module keeps the checkpoint's floating-point dtype
            if tuple(got.shape) != tuple(buf.shape):
                raise ValueError(f"{name}.{attr}: checkpoint shape {tuple(got.shape)} != declared {tuple(buf.shape)}")
            setattr(layer, attr, got.to(device))
        else:
            setattr(layer, attr, _coerce(f"{name}.{attr}", buf, got).to(device))
    if q is not None:
        m.process_weights_after_load(layer)
    return m, layer


def build_experts(quant: QuantConfig, prefix: str, num_experts: int, hidden: int, inter: int,
                  tensors: dict[str, torch.Tensor], *, device: str | torch.device = "cuda",
                  names: tuple[str, str, str] = ("gate_proj", "up_proj", "down_proj")):
    """(moe method, w13 container, w2 container) of routed experts `{prefix}.{e}.{gate,up,down}_proj`:
    gate|up merged per expert into w13 (2*inter outputs), down into w2, stacked over experts, then
    post_load (python/minisgl/layers/moe.py:42-407)."""
    q = quant.for_module(f"{prefix}.0.{names[0]}")
    moe = importlib.import_module(f"{_pkg}.layers.moe")
    mm = moe.create_moe_quant_method(q)
    w13 = mm.create_experts(num_experts, 2 * inter, hidden)
    w2 = mm.create_experts(num_experts, hidden, inter)
    nvfp4 = q.is_nvfp4
    for cont, parts in ((w13, names[:2]), (w2, names[2:])):
        for attr, buf in _declared(cont).items():
            per_expert = []
            for e in range(num_experts):
                pieces = [_fetch(tensors, f"{prefix}.{e}.{p}", attr, buf[0], nvfp4) for p in parts]
                ax = _n_axis(q, attr)
                per_expert.append(pieces[0] if len(pieces) == 1 or ax is None else torch.cat(pieces, dim=ax))
            got = torch.stack(per_expert)
            setattr(cont, attr, _coerce(f"{prefix}.*.{attr}", buf, got).to(device))
        cont.post_load()
    return mm, w13, w2
