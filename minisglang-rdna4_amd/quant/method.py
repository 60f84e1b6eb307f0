"""Linear quant methods for the W4A8 path: how a linear layer declares its checkpoint buffers,
converts them once after load, and runs its GEMM.

Mirrors the reference's method protocol and its W4A8 members (python/minisgl/quant/method.py):
LinearMethod (:352-364), W4A8LinearMethod (:384-574), MxFp4LinearMethod (:577-677),
NvFp4LinearMethod (:708-790),
create_linear_method (:680-705), the fused-SwiGLU shape gate _fused_swiglu_ok (:29-58) and the
compressed-tensors packed-sign decision (ct_packed_sign_convention / apply_ct_sign, :99-250).

Differences by design:
  * process_weights_after_load leaves the weight as W4 tiles (the gfx950 kernels' MFMA tile
    layout, still 4-bit) instead of the reference's (N, K/8) int32 op layout, so no call repacks;
    on a CPU-resident layer it stops at the op layout (the kernels accept both).
  * GPTQ's explicitly stored symmetric zero points (all 8) collapse to None: the kernels' symmetric
    path computes exactly the same values without reading a zero-point tensor.
  * The W4A16 arm (MINISGL_MOE_W4A16 != "0") runs the same weights through kernels.w4a16_linear;
    NVFP4 keeps its two-level scale (NvFp4LinearMethod). The fp8 methods are outside this package:
    create_linear_method raises NotImplementedError for those schemes.
"""
from __future__ import annotations

from typing import NamedTuple, Protocol

import torch
import torch.nn.functional as F

from . import kernels
from .config import QuantConfig


# ------------------------------------------------------------------------------------------------
# fused SwiGLU gate
# ------------------------------------------------------------------------------------------------
def _group_supported(group_size: int, k: int, weight_is_e2m1: bool = False) -> bool:
    g = int(group_size)
    ok = g in (32, 64) or (g >= 128 and (g & (g - 1)) == 0) or (g == 16 and weight_is_e2m1)
    return ok and k % g == 0


def _fused_swiglu_ok(x: torch.Tensor, w_packed: torch.Tensor, group_size: int, weight_is_e2m1: bool = False) -> bool:
    """Shape gate for the fused gate_up + silu decode GEMV (python/minisgl/quant/method.py:29-58):
    exactly the kernel's own constraints, no stricter -- decode rows (M <= 16), K % 32 == 0, a group
    size the kernel takes (32, 64 or a power of two >= 128 dividing K; 16, NVFP4's block, for e2m1
    weights), and N = 2 * inter with inter % 16 == 0 (whole 16-channel strips per half). No
    scale-format restriction: fp16, E8M0 and NVFP4 scales all reach the fused arm."""
    n = kernels._n_of(w_packed)
    k = x.shape[-1]
    return (x.dim() == 2 and x.shape[0] <= 16 and k % 32 == 0 and n % 32 == 0
            and _group_supported(group_size, k, weight_is_e2m1))


def _w4a16() -> bool:
    """The W4A16 arm (unquantized activations) is opt-in, as in the reference:
    MINISGL_MOE_W4A16 != "0" (python/minisgl/quant/kernels.py MOE_W4A16)."""
    return kernels.MOE_W4A16 != "0"


# ------------------------------------------------------------------------------------------------
# compressed-tensors packed sign convention
# ------------------------------------------------------------------------------------------------
_CT_SIGN_SAMPLE_WORDS = 1 << 16
_CT_SIGN_SAMPLE_BLOCKS = 512
_CT_SIGN_MIN_MARGIN = 1e-3


class CtSignConvention(NamedTuple):
    """The packed-nibble convention of one compressed-tensors int4 stack, decided once and reused
    for its weight and zero points (python/minisgl/quant/method.py:99-118)."""

    uint4b8: bool  # True: nibble = q + 8 already; False: two's complement (nibble = q & 0xF)
    margin: float
    sampled_words: int
    stride: int
    blocks: int = 1


def _ct_sign_sample(raw: torch.Tensor) -> tuple[torch.Tensor, int, int]:
    """At most _CT_SIGN_SAMPLE_WORDS packed words of the (n, elem) byte view, as
    _CT_SIGN_SAMPLE_BLOCKS contiguous runs spread evenly over the whole tensor (first run at 0,
    last ending at n) -- never a prefix, never a lattice that could alias a row length."""
    n = int(raw.shape[0])
    if n <= _CT_SIGN_SAMPLE_WORDS:
        return raw, 1, 1
    blocks = _CT_SIGN_SAMPLE_BLOCKS
    run = max(1, _CT_SIGN_SAMPLE_WORDS // blocks)
    last = n - run
    step = last // (blocks - 1)
    first = torch.arange(blocks, dtype=torch.int64, device=raw.device) * last // (blocks - 1)
    idx = (first[:, None] + torch.arange(run, dtype=torch.int64, device=raw.device)[None, :]).reshape(-1)
    return raw.index_select(0, idx), blocks, step


def ct_packed_sign_convention(packed: torch.Tensor, *, name: str = "weight_packed",
                              min_margin: float = _CT_SIGN_MIN_MARGIN) -> CtSignConvention:
    """Decide uint4b8 (mode of the nibble histogram at 8) vs two's complement (mode at 0) from a
    whole-tensor sample (python/minisgl/quant/method.py:143-224). An ambiguous histogram raises
    ValueError instead of guessing, since a wrong guess flips every nibble silently."""
    if packed.numel() == 0:
        raise ValueError(f"{name}: empty packed tensor, no sign convention to decide")
    elem = packed.element_size()
    raw = packed.contiguous().view(torch.uint8).reshape(-1, elem)
    n = int(raw.shape[0])
    sample, blocks, stride = _ct_sign_sample(raw)
    s16 = sample.to(torch.int16)
    nib = torch.cat([s16 & 0xF, (s16 >> 4) & 0xF]).reshape(-1).to(torch.int64)
    counts = torch.bincount(nib, minlength=16)
    c8, c0 = int(counts[8]), int(counts[0])
    total = int(nib.numel())
    margin = abs(c8 - c0) / total if total else 0.0
    if margin < min_margin:
        raise ValueError(
            f"{name}: cannot decide the compressed-tensors int4 packing: sampled {int(sample.shape[0])} of {n} "
            f"packed {elem * 8}-bit words ({blocks} block(s), stride {stride}); nibble counts at 8 and 0 are {c8} "
            f"and {c0} (margin {margin:.2e} < {min_margin:.0e}). uint4b8 and two's complement are "
            f"indistinguishable here; inspect the checkpoint's quantization_config.")
    return CtSignConvention(uint4b8=c8 > c0, margin=margin, sampled_words=int(sample.shape[0]),
                            stride=stride, blocks=blocks)


def apply_ct_sign(t: torch.Tensor, conv: CtSignConvention) -> torch.Tensor:
    """Bring a packed int4 tensor into the kernels' uint4b8 domain under a decided convention:
    two's complement becomes q + 8 by flipping each nibble's top bit (XOR 0x88 per byte); uint4b8
    passes through. Dtype-preserving (python/minisgl/quant/method.py:226-245)."""
    t = t.contiguous()
    if conv.uint4b8:
        return t
    return (t.view(torch.uint8) ^ 0x88).view(t.dtype)


# ------------------------------------------------------------------------------------------------
# methods
# ------------------------------------------------------------------------------------------------
class LinearMethod(Protocol):
    """How a linear layer allocates its weights and computes its matmul
    (python/minisgl/quant/method.py:352-364)."""

    def create_weights(self, layer, out_features: int, in_features: int) -> None: ...

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor: ...


class UnquantizedLinearMethod:
    """bf16/fp16 dense linear (layers the checkpoint leaves unquantized, e.g. lm_head)."""

    def create_weights(self, layer, out_features: int, in_features: int) -> None:
        layer.weight = torch.empty(out_features, in_features)

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        return F.linear(x, layer.weight, bias)


def _to_kernel_layout(w_op: torch.Tensor, weight_is_e2m1: bool) -> torch.Tensor:
    """Op layout -> W4 tiles on a GPU-resident layer (one repack at load); CPU layers keep the op
    layout, which the kernels also accept."""
    return kernels.repack_w4(w_op, weight_is_e2m1) if w_op.is_cuda else w_op


def _drop_symmetric_zeros(zeros: torch.Tensor | None) -> torch.Tensor | None:
    """Zero points that are all 8 (GPTQ stores the symmetric zero explicitly) -> None."""
    if zeros is None:
        return None
    if bool((zeros.view(torch.uint8) == 0x88).all()):
        return None
    return zeros


class W4A8LinearMethod:
    """int4 weight x per-token fp8 activation linear (python/minisgl/quant/method.py:384-574).

    Buffers are declared in CHECKPOINT layout (shapes and dtypes match the file exactly), converted
    to the kernels' layout once in process_weights_after_load:
      GPTQ: qweight (K/8, N) i32, scales (K/g, N) f16, qzeros (K/g, N/8) i32 (+ g_idx with desc_act)
      AWQ:  qweight (K, N/8) i32, scales (K/g, N) f16, qzeros (K/g, N/8) i32 when asymmetric
      compressed-tensors int4: weight_packed (N, K/8) i32, weight_scale (N, K/g) f16,
            weight_zero_point (N/8, K/g) i32 when asymmetric."""

    def __init__(self, quant: QuantConfig) -> None:
        self.quant = quant

    @property
    def supports_producer_actquant(self) -> bool:
        # the W4A16 arm reads x unquantized: a producer fp8 pair has nothing to feed
        return not _w4a16()

    def create_weights(self, layer, out_features: int, in_features: int) -> None:
        pf = 32 // self.quant.bits
        g = self.quant.group_size
        N, K = out_features, in_features
        if self.quant.is_gptq:
            assert K % pf == 0 and K % g == 0 and N % pf == 0, f"GPTQ needs K%{pf}==0,K%{g}==0,N%{pf}==0; got N={N},K={K}"
            layer.qweight = torch.empty((K // pf, N), dtype=torch.int32)
            layer.scales = torch.empty((K // g, N), dtype=torch.float16)
            layer.qzeros = torch.empty((K // g, N // pf), dtype=torch.int32)
            if self.quant.desc_act:
                layer.g_idx = torch.empty((K,), dtype=torch.int32)
            return
        if self.quant.is_compressed_tensors:
            assert K % pf == 0 and K % g == 0 and N % pf == 0, (
                f"CT dense needs K%{pf}==0,K%{g}==0,N%{pf}==0; got N={N},K={K}")
            layer.weight_packed = torch.empty((N, K // pf), dtype=torch.int32)
            layer.weight_scale = torch.empty((N, K // g), dtype=torch.float16)
            if not self.quant.sym:
                layer.weight_zero_point = torch.empty((N // pf, K // g), dtype=torch.int32)
            return
        assert N % pf == 0 and K % g == 0, f"W4A8 needs N%{pf}==0,K%{g}==0; got N={N},K={K}"
        layer.qweight = torch.empty((K, N // pf), dtype=torch.int32)
        layer.scales = torch.empty((K // g, N), dtype=torch.float16)
        if not self.quant.sym:
            layer.qzeros = torch.empty((K // g, N // pf), dtype=torch.int32)

    def process_weights_after_load(self, layer) -> None:
        if self.quant.is_compressed_tensors:
            wp = layer.weight_packed.contiguous()
            conv = ct_packed_sign_convention(wp, name=f"{type(layer).__name__}.weight_packed")
            layer._ct_sign = conv
            w_op = apply_ct_sign(wp, conv)  # (N, K/8): nibble j of word k/8 is input k, uint4b8
            layer._scales_op = layer.weight_scale.to(torch.float16).transpose(0, 1).contiguous()  # (K/g, N)
            zp = getattr(layer, "weight_zero_point", None)
            if zp is None:
                layer._zeros_op = None
            else:
                # packed 8 channels per word along N within each int32: transposing (N/8, G) is exact
                layer._zeros_op = apply_ct_sign(zp.contiguous(), conv).transpose(0, 1).contiguous()
                del layer.weight_zero_point
            layer._w_packed_op = _to_kernel_layout(w_op, False)
            del layer.weight_packed, layer.weight_scale
            return
        qz = getattr(layer, "qzeros", None)
        if self.quant.is_gptq:
            assert not self.quant.desc_act, "GPTQ desc_act (act-order) not supported"
            w_op, s_op, z_op = kernels.gptq_to_op_layout(layer.qweight, layer.scales, qz, bits=self.quant.bits)
        else:
            w_op, s_op, z_op = kernels.awq_to_op_layout(layer.qweight, layer.scales, qz, bits=self.quant.bits)
        layer._w_packed_op = _to_kernel_layout(w_op, False)
        layer._scales_op = s_op
        layer._zeros_op = _drop_symmetric_zeros(z_op)
        del layer.qweight, layer.scales
        if qz is not None:
            del layer.qzeros

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None, *,
              x_fp8: torch.Tensor | None = None, act_scales: torch.Tensor | None = None) -> torch.Tensor:
        if _w4a16():
            out = kernels.w4a16_linear(x, layer._w_packed_op, layer._scales_op, layer._zeros_op, self.quant.group_size,
                                       kernels._n_of(layer._w_packed_op))
        else:
            out = kernels.w4a8_linear(x, layer._w_packed_op, layer._scales_op, layer._zeros_op, self.quant.group_size,
                                      x_fp8=x_fp8, act_scales=act_scales)
        out = out.to(x.dtype)
        if bias is not None:
            out = out + bias
        return out

    def apply_swiglu(self, layer, x: torch.Tensor) -> torch.Tensor | None:
        """Fused gate_up + silu at decode on a merged gate_up layer; None -> the caller runs the
        unfused pair. Bit-exact to the unfused pair when it fires."""
        w = layer._w_packed_op
        if not _fused_swiglu_ok(x, w, self.quant.group_size):
            return None
        fn = kernels.w4a16_linear_silu if _w4a16() else kernels.w4a8_linear_silu
        return fn(x, w, layer._scales_op, layer._zeros_op, self.quant.group_size).to(x.dtype)


class MxFp4LinearMethod:
    """MXFP4 (E2M1 codes + E8M0 per-32 block scale) linear through the same W4A8 kernels with
    weight_is_e2m1=True (python/minisgl/quant/method.py:577-677). Checkpoint layout:
    weight_packed (N, K/2) uint8 (two E2M1 nibbles per byte, low nibble = lower K), weight_scale
    (N, K/32) uint8 E8M0. The E8M0 bytes reach the MFMA unchanged."""

    def __init__(self, quant: QuantConfig) -> None:
        self.quant = quant

    @property
    def supports_producer_actquant(self) -> bool:
        return not _w4a16()

    def create_weights(self, layer, out_features: int, in_features: int) -> None:
        N, K = out_features, in_features
        g = self.quant.group_size
        assert K % 2 == 0 and K % g == 0 and N % 8 == 0, f"MXFP4 needs K%2==0,K%{g}==0,N%8==0; got N={N},K={K}"
        layer.weight_packed = torch.empty((N, K // 2), dtype=torch.uint8)
        layer.weight_scale = torch.empty((N, K // g), dtype=torch.uint8)

    def process_weights_after_load(self, layer) -> None:
        from . import mxfp4

        conv = mxfp4.convert_mxfp4_weight(layer.weight_packed, layer.weight_scale)
        layer._scale_info = conv["scale_info"]
        layer._w_packed_op = _to_kernel_layout(conv["w_packed"], True)
        layer._scales_op = conv["scales"].transpose(0, 1).contiguous()  # (K/32, N) E8M0, group-major
        del layer.weight_packed, layer.weight_scale

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None, *,
              x_fp8: torch.Tensor | None = None, act_scales: torch.Tensor | None = None) -> torch.Tensor:
        if _w4a16():
            out = kernels.w4a16_linear(x, layer._w_packed_op, layer._scales_op, None, self.quant.group_size,
                                       kernels._n_of(layer._w_packed_op), weight_is_e2m1=True)
        else:
            out = kernels.w4a8_linear(x, layer._w_packed_op, layer._scales_op, None, self.quant.group_size,
                                      weight_is_e2m1=True, x_fp8=x_fp8, act_scales=act_scales)
        out = out.to(x.dtype)
        if bias is not None:
            out = out + bias
        return out

    def apply_swiglu(self, layer, x: torch.Tensor) -> torch.Tensor | None:
        w = getattr(layer, "_w_packed_op", None)
        if w is None or not _fused_swiglu_ok(x, w, self.quant.group_size, weight_is_e2m1=True):
            return None
        fn = kernels.w4a16_linear_silu if _w4a16() else kernels.w4a8_linear_silu
        return fn(x, w, layer._scales_op, None, self.quant.group_size, weight_is_e2m1=True).to(x.dtype)


class NvFp4LinearMethod:
    """NVFP4 dense linear (python/minisgl/quant/method.py:708-790): the e2m1 kernels with the
    two-level scale kept as two levels. Checkpoint-native buffers: weight_packed (N, K/2) uint8 (two
    E2M1 nibbles per byte, low nibble = lower K), weight_scale (N, K/16) float8_e4m3fn block scales
    (byte-verbatim), weight_global (N,) f32 per-output-channel multiplier (the loader's
    nvfp4.split_nvfp4_scale output, direction already normalised). After load: W4 tiles, group-major
    (K/16, N) e4m3 scales and the global's f32 bits as int32 for the zeros slot."""

    def __init__(self, quant: QuantConfig) -> None:
        self.quant = quant

    @property
    def supports_producer_actquant(self) -> bool:
        return not _w4a16()

    def create_weights(self, layer, out_features: int, in_features: int) -> None:
        N, K = out_features, in_features
        g = self.quant.group_size
        assert g == 16, f"NVFP4 blocks are 16 elements; got group_size={g}"
        assert K % 32 == 0 and N % 16 == 0, f"NVFP4 needs K%32==0,N%16==0; got N={N},K={K}"
        layer.weight_packed = torch.empty((N, K // 2), dtype=torch.uint8)
        layer.weight_scale = torch.empty((N, K // g), dtype=torch.float8_e4m3fn)
        layer.weight_global = torch.empty((N,), dtype=torch.float32)

    def process_weights_after_load(self, layer) -> None:
        from . import nvfp4

        conv = nvfp4.convert_nvfp4_weight(layer.weight_packed, layer.weight_scale)
        layer._w_packed_op = _to_kernel_layout(conv["w_packed"], True)
        layer._scales_op = conv["scales"].transpose(0, 1).contiguous()  # (K/16, N) e4m3, group-major
        # the f32 bits viewed as int32 (a value conversion would truncate every global to 0)
        layer._global_op = layer.weight_global.to(torch.float32).contiguous().view(torch.int32)
        del layer.weight_packed, layer.weight_scale, layer.weight_global

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None, *,
              x_fp8: torch.Tensor | None = None, act_scales: torch.Tensor | None = None) -> torch.Tensor:
        if _w4a16():
            out = kernels.w4a16_linear(x, layer._w_packed_op, layer._scales_op, layer._global_op, 16,
                                       kernels._n_of(layer._w_packed_op), weight_is_e2m1=True)
        else:
            out = kernels.w4a8_linear(x, layer._w_packed_op, layer._scales_op, layer._global_op, 16,
                                      weight_is_e2m1=True, x_fp8=x_fp8, act_scales=act_scales)
        out = out.to(x.dtype)
        if bias is not None:
            out = out + bias
        return out

    def apply_swiglu(self, layer, x: torch.Tensor) -> torch.Tensor | None:
        w = getattr(layer, "_w_packed_op", None)
        if w is None or not _fused_swiglu_ok(x, w, 16, weight_is_e2m1=True):
            return None
        fn = kernels.w4a16_linear_silu if _w4a16() else kernels.w4a8_linear_silu
        return fn(x, w, layer._scales_op, layer._global_op, 16, weight_is_e2m1=True).to(x.dtype)


def create_linear_method(quant: QuantConfig | None, *, quantized: bool = True):
    """Pick the method for a linear layer from the declared scheme
    (python/minisgl/quant/method.py:680-705); quantized=False keeps a layer unquantized."""
    if quant is None or not quantized:
        return UnquantizedLinearMethod()
    if quant.is_nvfp4:
        return NvFp4LinearMethod(quant)
    if quant.weight_is_e2m1:
        return MxFp4LinearMethod(quant)
    if quant.is_fp8_block or quant.is_fp8_w8a8:
        raise NotImplementedError("fp8 W8A8 linears are not served by this W4A8 path")
    if not quant.is_int4:
        raise AssertionError(f"unsupported declared quant scheme (method={quant.method}, bits={quant.bits}, "
                             f"weight_type={quant.weight_type})")
    return W4A8LinearMethod(quant)
