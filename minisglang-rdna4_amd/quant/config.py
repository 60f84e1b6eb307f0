"""Declared quantization scheme of a checkpoint, as the W4A8 methods read it.

Mirrors the fields and predicates of the reference's QuantConfig (python/minisgl/quant/config.py:
294-418) that the W4A8 hot path dispatches on: method / bits / group_size / sym / desc_act /
weight_type / ct_format and the is_awq, is_gptq, is_compressed_tensors, is_int4, weight_is_e2m1,
is_nvfp4, is_fp8_w8a8, is_fp8_block predicates. Parsing a HuggingFace quantization_config into this
object (the reference's from_hf, config.py:494-622) is checkpoint ingestion and is not part of this
package; callers construct the object directly.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class QuantConfig:
    method: str  # "awq" | "gptq" | "compressed-tensors"
    bits: int  # 4 for the W4A8 family
    group_size: int  # 128 (AWQ/GPTQ), 32 (compressed-tensors int4, MXFP4)
    sym: bool  # symmetric (zero point 8) vs asymmetric (per-group zero points)
    desc_act: bool = False  # GPTQ act-order; not supported by the W4A8 layouts
    weight_type: str = "int"  # "int" (int4) | "float" (E2M1 for 4-bit)
    ct_format: str | None = None  # compressed-tensors format, e.g. "mxfp4-pack-quantized"
    weight_strategy: str | None = None
    block_structure: tuple[int, ...] | None = None

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
