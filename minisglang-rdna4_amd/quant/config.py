"""Declared quantization scheme of a checkpoint, as the W4A8 methods read it.

Mirrors the fields and predicates of the reference's QuantConfig (python/minisgl/quant/config.py:
294-492): method / bits / group_size / sym / desc_act / weight_type / ct_format, the is_awq,
is_gptq, is_compressed_tensors, is_int4, weight_is_e2m1, is_nvfp4, is_fp8_w8a8, is_fp8_block
predicates, the module filter (is_module_quantized, for_module) and QuantConfig.from_hf
(config.py:494-622), which reads a HuggingFace quantization_config:
  * awq  -> asymmetric unless zero_point is false; gptq -> sym / desc_act as declared;
    modules_to_not_convert become plain ignore entries;
  * compressed-tensors -> the first config group's weights block (num_bits, group_size,
    symmetric, type, strategy, block_structure) plus the top-level format; several groups (or
    format "mixed-precision") are all kept, class-name targets ("Linear") treated as catch-alls
    and ordered last, and for_module picks the first group whose targets match;
  * modelopt (NVFP4 / FP8 headers) is rewritten into the compressed-tensors shape first, glob
    ignore entries becoming anchored regexes;
  * AMD Quark (config.py:228-293, called at :515) is rewritten the same way: the weight format is
    the (dtype, scale_format) pair of global_quant_config.weight, looked up in a closed table, and
    `exclude` names parameter tensors, so their `.weight` / `.bias` / `.weight_scale` suffix is cut
    to the module name the ignore match uses. Dynamic weight quant, per-layer override tables and
    any on-disk packing other than "reorder" are refused (None): each would load without error and
    compute wrong numbers.
Other methods give None: the checkpoint is not one these kernels serve.
"""
from __future__ import annotations

import dataclasses
import fnmatch
import re
from dataclasses import dataclass
from typing import Any


def _norm_ignore(patterns) -> tuple[str, ...]:
    """Checkpoint-space ignore entries -> the loader's module names: the multimodal
    'language_model.' infix and a leading 'model.decoder.' are stripped from plain entries
    (config.py:10-30); 're:' regexes are left as written."""
    out = []
    for p in patterns or ():
        p = str(p)
        if p and not p.startswith("re:"):
            p = p.replace("language_model.", "")
            if p.startswith("model.decoder."):
                p = "model." + p[len("model.decoder."):]
        out.append(p)
    return tuple(out)


_GLOB = ("*", "?", "[")


def _glob_to_ignore(p: str) -> str:
    """A modelopt glob becomes an anchored regex; a plain name keeps substring semantics."""
    if p.startswith("re:") or not any(c in p for c in _GLOB):
        return p
    return "re:" + r"\A" + fnmatch.translate(p)


_MODELOPT_FORMAT = {"NVFP4": "nvfp4-pack-quantized", "NVFP4_AWQ": "nvfp4-pack-quantized",
                    "FP8": "float-quantized", "FP8_PER_TENSOR": "float-quantized",
                    "FP8_PER_CHANNEL_PER_TOKEN": "float-quantized"}
_MODELOPT_SCHEME = {
    "nvfp4-pack-quantized": {"weights": {"num_bits": 4, "group_size": 16, "type": "float", "symmetric": True},
                             "input_activations": {"num_bits": 4, "type": "float"}},
    "float-quantized": {"weights": {"num_bits": 8, "type": "float", "symmetric": True},
                        "input_activations": {"num_bits": 8, "type": "float"}},
}


def _modelopt_to_ct(d: dict) -> dict | None:
    """modelopt header -> compressed-tensors shape (config.py:114-150), None for an unknown algo."""
    algo = str(d.get("quant_algo") or "").upper()
    fmt = _MODELOPT_FORMAT.get(algo)
    if fmt is None:
        return None
    groups = d.get("config_groups") or {}
    if not any((g or {}).get("weights") for g in groups.values()):
        groups = {"group_0": dict(_MODELOPT_SCHEME[fmt], targets=("re:.*",))}
    else:
        def tgt(t):
            t = str(t)
            return "re:.*" if (t and "." not in t and not any(c in t for c in _GLOB)) else _glob_to_ignore(t)
        groups = {k: dict(g, targets=tuple(tgt(t) for t in (g.get("targets") or ()))) for k, g in groups.items()}
    return {"quant_method": "compressed-tensors", "format": fmt, "config_groups": groups,
            "ignore": tuple(_glob_to_ignore(p) for p in _norm_ignore(d.get("ignore") or ()))}


# Quark weight (dtype, scale_format) -> the compressed-tensors format with the same on-disk layout.
# Closed: a pair not listed is a packing no reader here understands, and is refused.
_QUARK_FORMAT = {
    ("fp4", "e8m0"): "mxfp4-pack-quantized",   # E2M1 codes, E8M0 block exponents
    ("fp4", "e4m3"): "nvfp4-pack-quantized",   # E2M1 codes, e4m3 block scales, per-tensor global
    ("fp8_e4m3", "float"): "float-quantized",
    ("fp8_e4m3", ""): "float-quantized",
}
_QUARK_PACKINGS = ("reorder",)  # the nibble order the compressed-tensors readers expect
_PARAM_SUFFIXES = (".weight", ".bias", ".weight_scale")


def _strip_param_suffix(name: str) -> str:
    for sfx in _PARAM_SUFFIXES:
        if name.endswith(sfx):
            return name[: -len(sfx)]
    return name


def _quark_to_ct(d: dict) -> dict | None:
    """Quark header -> compressed-tensors shape (config.py:228-293), None when it is refused."""
    gq = d.get("global_quant_config") or {}
    w = gq.get("weight") or gq.get("weights") or {}
    dt = str(w.get("dtype") or "").lower()
    fmt = _QUARK_FORMAT.get((dt, str(w.get("scale_format") or "").lower()))
    if fmt is None or w.get("is_dynamic"):
        return None
    if d.get("layer_quant_config") or d.get("layer_type_quant_config"):
        return None  # per-layer overrides: no reader for a per-layer mixed scheme
    packing = str((d.get("export") or {}).get("pack_method") or "reorder").lower()
    if packing not in _QUARK_PACKINGS:
        return None
    weights = {"num_bits": 4 if dt == "fp4" else 8, "type": "float", "strategy": "group",
               "group_size": int(w.get("group_size") or 32), "symmetric": True}
    return {"quant_method": "compressed-tensors", "format": fmt,
            # the checkpoint's activation scheme is not consumed: the methods pick per-token fp8
            # (W4A8) or unquantized (W4A16), as for a compressed-tensors file declaring none
            "config_groups": {"group_0": {"targets": ["Linear"], "weights": weights, "input_activations": None}},
            "ignore": _norm_ignore(_strip_param_suffix(str(e)) for e in (d.get("exclude") or ()))}


def _targets(targets) -> tuple[tuple[str, ...], bool]:
    """Group targets -> (patterns, is catch-all): a bare class name such as "Linear" selects every
    linear, i.e. 're:.*' (config.py:183-210)."""
    out, catchall = [], False
    for t in targets or ():
        t = str(t)
        if not t.startswith("re:") and "." not in t and "/" not in t and t[:1].isupper() and t.isidentifier():
            out.append("re:.*")
            catchall = True
        else:
            out.append(t)
    return tuple(out), catchall


@dataclass(frozen=True)
class QuantConfig:
    method: str  # "awq" | "gptq" | "compressed-tensors"
    bits: int  # 4 for the W4A8 family
    group_size: int  # 128 (AWQ/GPTQ), 32 (compressed-tensors int4, MXFP4), 16 (NVFP4)
    sym: bool  # symmetric (zero point 8) vs asymmetric (per-group zero points)
    desc_act: bool = False  # GPTQ act-order; not supported by the W4A8 layouts
    weight_type: str = "int"  # "int" (int4) | "float" (E2M1 for 4-bit)
    ct_format: str | None = None  # compressed-tensors format, e.g. "mxfp4-pack-quantized"
    weight_strategy: str | None = None
    block_structure: tuple[int, ...] | None = None
    ignore: tuple[str, ...] = ()  # modules kept unquantized ('re:' regex or plain substring)
    act_type: str | None = None  # "fp8" when input activations are declared (W8A8 schemes)
    # mixed precision: ((target patterns), scheme) per config group, first match wins
    ct_groups: tuple = ()

    @property
    def is_awq(self) -> bool:
        return self.method == "awq"

    @property
    def is_gptq(self) -> bool:
        return self.method == "gptq"

    @property
    def is_compressed_tensors(self) -> bool:
        return self.method == "compressed-tensors"

    @property
    def is_fp8_w8a8(self) -> bool:
        return self.is_compressed_tensors and self.weight_type == "float" and self.bits == 8

    @property
    def is_fp8_block(self) -> bool:
        return self.is_fp8_w8a8 and self.weight_strategy == "block" and bool(self.block_structure)

    @property
    def is_nvfp4(self) -> bool:
        return self.is_compressed_tensors and self.ct_format == "nvfp4-pack-quantized"

    @property
    def weight_is_e2m1(self) -> bool:
        """MXFP4: compressed-tensors float-quantized 4-bit (E2M1 codes, E8M0 block-32 scales)."""
        return self.is_compressed_tensors and self.weight_type == "float" and self.bits == 4 and not self.is_nvfp4

    @property
    def is_int4(self) -> bool:
        return self.bits == 4 and self.weight_type == "int"

    # ---------------------------------------------------------------- module filter
    def is_module_quantized(self, name: str, *, exact: bool = False) -> bool:
        """False when `name` matches an ignore entry: a 're:' regex searched in the name, or a
        plain entry as a substring (exact=True: the entry must end the name at a dot boundary)
        (config.py:418-444)."""
        for pat in self.ignore:
            if not pat:
                continue
            if pat.startswith("re:"):
                if re.search(pat[3:], name):
                    return False
            elif (name == pat or name.endswith("." + pat)) if exact else (pat in name):
                return False
        return True

    def for_module(self, name: str) -> "QuantConfig | None":
        """The scheme module `name` is quantized with, or None when it is kept unquantized: ignored
        modules give None; with several config groups the first group whose targets match wins and a
        module no group selects is unquantized (config.py:446-484)."""
        if not self.is_module_quantized(name, exact=bool(self.ct_groups)):
            return None
        if not self.ct_groups:
            return self
        for targets, scheme in self.ct_groups:
            for pat in targets:
                if pat and ((pat.startswith("re:") and re.search(pat[3:], name)) or
                            (not pat.startswith("re:") and pat in name)):
                    return scheme
        return None

    # ---------------------------------------------------------------- HuggingFace header
    @staticmethod
    def _as_dict(qc: Any) -> dict:
        if isinstance(qc, dict):
            return qc
        if hasattr(qc, "to_dict"):
            return qc.to_dict()
        return dict(getattr(qc, "__dict__", {}))

    @classmethod
    def from_hf(cls, hf_config: Any) -> "QuantConfig | None":
        """The scheme a HuggingFace config declares (its quantization_config, or text_config's), or
        None when there is none or it is not a W4A8-family header (config.py:494-622)."""
        get = (lambda o, k: o.get(k)) if isinstance(hf_config, dict) else (lambda o, k: getattr(o, k, None))
        qc = get(hf_config, "quantization_config")
        if qc is None and get(hf_config, "text_config") is not None:
            tc = get(hf_config, "text_config")
            qc = tc.get("quantization_config") if isinstance(tc, dict) else getattr(tc, "quantization_config", None)
        if qc is None:
            return None
        d = cls._as_dict(qc)
        method = str(d.get("quant_method", "")).lower()
        if method in ("modelopt", "modelopt_fp8", "modelopt_fp4"):
            d = _modelopt_to_ct(d)
            if d is None:
                return None
            method = "compressed-tensors"
        if method == "quark":
            d = _quark_to_ct(d)
            if d is None:
                return None
            method = "compressed-tensors"
        not_convert = _norm_ignore(d.get("modules_to_not_convert") or ())
        if method == "awq":
            return cls(method="awq", bits=int(d.get("bits", 4)), group_size=int(d.get("group_size", 128)),
                       sym=not bool(d.get("zero_point", True)), ignore=not_convert)
        if method == "gptq":
            return cls(method="gptq", bits=int(d.get("bits", 4)), group_size=int(d.get("group_size", 128)),
                       sym=bool(d.get("sym", True)), desc_act=bool(d.get("desc_act", False)), ignore=not_convert)
        if method not in ("compressed-tensors", "compressed_tensors"):
            return None
        fmt = str(d.get("format", "")).lower() or None
        ignore = _norm_ignore(d.get("ignore") or ())

        def scheme(g: dict, group_fmt: str | None) -> QuantConfig:
            w = (g or {}).get("weights") or {}
            ia = (g or {}).get("input_activations") or {}
            own = str((g or {}).get("format", "")).lower() or None
            if own is None and str(w.get("type", "")).lower() == "float" and int(w.get("num_bits") or 0) == 8:
                own = "float-quantized"  # 8-bit float is fp8 whatever the headline format says
            return cls(method="compressed-tensors",
                       bits=int(w["num_bits"]) if w.get("num_bits") else 4,
                       group_size=int(w["group_size"]) if w.get("group_size") else 32,
                       sym=bool(w["symmetric"]) if w.get("symmetric") is not None else True,
                       weight_type=str(w["type"]).lower() if w.get("type") else "int",
                       ct_format=own or group_fmt,
                       weight_strategy=str(w["strategy"]).lower() if w.get("strategy") else None,
                       block_structure=tuple(int(b) for b in w["block_structure"]) if w.get("block_structure") else None,
                       ignore=ignore,
                       act_type="fp8" if ia and str(ia.get("type", "")).lower() == "float" and
                       int(ia.get("num_bits") or 8) == 8 else None)

        ordered = [g for g in (d.get("config_groups") or {}).values() if (g or {}).get("weights")]
        groups = ()
        if len(ordered) > 1 or fmt == "mixed-precision":
            parsed = [(_norm_ignore(pats), scheme(g, fmt), catchall)
                      for g in ordered for pats, catchall in (_targets(g.get("targets")),)]
            groups = tuple((p, sc) for p, sc, ca in parsed if not ca) + tuple((p, sc) for p, sc, ca in parsed if ca)
        head = scheme(ordered[0], fmt) if ordered else cls(method="compressed-tensors", bits=4, group_size=32,
                                                          sym=True, ignore=ignore)
        # the headline keeps the first group's scalars and the top-level format (config.py:618-621)
        return dataclasses.replace(head, ct_format=fmt, ct_groups=groups)
