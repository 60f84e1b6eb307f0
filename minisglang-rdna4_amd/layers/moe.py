"""MoE expert containers and quant methods for the W4A8 path.

Mirrors the reference's expert storage and method layer (python/minisgl/layers/moe.py):
_GroupedGPTQExperts (:42-95), _GroupedAWQExperts (:97-145), _GroupedCompressedTensorsExperts
(:147-266), _GroupedMxFp4Experts (:268-343), the MoEQuantMethod protocol (:520-580),
_W4A8MoEMethod (:623-709), _MxFp4MoEMethod (:712-788) and create_moe_quant_method (:971-1005).
Routing, EP dispatch/combine and TP reduction belong to the MoE layer around these and are not
part of this package; ep_local is the per-rank kernel call over a local expert shard with a
precomputed route.

Containers declare CHECKPOINT-layout buffers stacked over E on dim 0; post_load converts each
expert to the op layout and, on a GPU-resident container, to W4 tiles (one repack at load, none per
call). Zero points that are all 8 collapse to None (the kernels' symmetric path is exact for them).
"""
from __future__ import annotations

import importlib
import logging

import torch

_pkg = __name__.rsplit(".", 2)[0]
kernels = importlib.import_module(f"{_pkg}.quant.kernels")
_method = importlib.import_module(f"{_pkg}.quant.method")


def _finish(w_op: torch.Tensor, weight_is_e2m1: bool) -> torch.Tensor:
    return kernels.repack_w4(w_op, weight_is_e2m1) if w_op.is_cuda else w_op


class _GroupedGPTQExperts:
    """GPTQ experts for one MoE GEMM (w13 or w2), N = out, K = in per expert:
    qweight (E, K/8, N) i32, scales (E, K/g, N) f16, qzeros (E, K/g, N/8) i32. After post_load:
    _w_op (E, N/16, ceil(K/128), 1024) W4 tiles, _scales_op (E, K/g, N), _zeros_op (E, K/g, N/8)
    or None."""

    def __init__(self, num_experts: int, out_features: int, in_features: int, quant):
        pf = 32 // quant.bits
        g = quant.group_size
        N, K = out_features, in_features
        assert K % pf == 0 and K % g == 0 and N % pf == 0, (
            f"grouped GPTQ needs K%{pf}==0,K%{g}==0,N%{pf}==0; got N={N},K={K}")
        self.qweight = torch.empty((num_experts, K // pf, N), dtype=torch.int32)
        self.scales = torch.empty((num_experts, K // g, N), dtype=torch.float16)
        self.qzeros = torch.empty((num_experts, K // g, N // pf), dtype=torch.int32)
        self._quant = quant
        self._num_experts = num_experts

    def forward(self, *args, **kwargs):
        raise RuntimeError(f"{type(self).__name__} holds weights; call kernels.w4a8_moe instead")

    def _convert(self, fn) -> None:
        E = self.qweight.shape[0]
        parts = [fn(self.qweight[e], self.scales[e], self.qzeros[e] if self.qzeros is not None else None,
                    bits=self._quant.bits) for e in range(E)]
        self._w_op = _finish(torch.stack([p[0] for p in parts]), False)
        self._scales_op = torch.stack([p[1] for p in parts])
        z = None if parts[0][2] is None else torch.stack([p[2] for p in parts])
        self._zeros_op = _method._drop_symmetric_zeros(z)
        del self.qweight, self.scales, self.qzeros

    def post_load(self) -> None:
        assert not self._quant.desc_act, "GPTQ desc_act (act-order) not supported"
        self._convert(kernels.gptq_to_op_layout)


class _GroupedAWQExperts(_GroupedGPTQExperts):
    """AWQ-gemm experts: qweight (E, K, N/8) i32 (packed along N with the AWQ interleave), scales
    (E, K/g, N) f16, qzeros (E, K/g, N/8) i32 (AWQ is asymmetric: zeros always present)."""

    def __init__(self, num_experts: int, out_features: int, in_features: int, quant):
        pf = 32 // quant.bits
        g = quant.group_size
        N, K = out_features, in_features
        assert N % pf == 0 and K % g == 0, f"AWQ experts need N%{pf}==0,K%{g}==0; got N={N},K={K}"
        self.qweight = torch.empty((num_experts, K, N // pf), dtype=torch.int32)
        self.scales = torch.empty((num_experts, K // g, N), dtype=torch.float16)
        self.qzeros = torch.empty((num_experts, K // g, N // pf), dtype=torch.int32)
        self._quant = quant
        self._num_experts = num_experts

    def post_load(self) -> None:
        self._convert(kernels.awq_to_op_layout)


class _GroupedCompressedTensorsExperts:
    """compressed-tensors int4 experts: weight_packed (E, N, K/8) i32 (natural K order),
    weight_scale (E, N, K/g) f16, weight_zero_point (E, N/8, K/g) i32 when asymmetric. The packed
    sign convention is decided once per stack and applied to weight and zero points alike."""

    def __init__(self, num_experts: int, out_features: int, in_features: int, quant):
        pf = 32 // quant.bits
        g = quant.group_size
        N, K = out_features, in_features
        assert K % pf == 0 and K % g == 0 and N % pf == 0, (
            f"grouped compressed-tensors needs K%{pf}==0,K%{g}==0,N%{pf}==0; got N={N},K={K}")
        self.weight_packed = torch.empty((num_experts, N, K // pf), dtype=torch.int32)
        self.weight_scale = torch.empty((num_experts, N, K // g), dtype=torch.float16)
        if not quant.sym:
            self.weight_zero_point = torch.empty((num_experts, N // pf, K // g), dtype=torch.int32)
        self._quant = quant
        self._num_experts = num_experts

    def forward(self, *args, **kwargs):
        raise RuntimeError(f"{type(self).__name__} holds weights; call kernels.w4a8_moe instead")

    def post_load(self) -> None:
        wp = self.weight_packed.contiguous()
        conv = _method.ct_packed_sign_convention(wp, name=f"{type(self).__name__}.weight_packed")
        self._ct_sign = conv
        self._w_op = _finish(_method.apply_ct_sign(wp, conv), False)
        self._scales_op = self.weight_scale.to(torch.float16).transpose(1, 2).contiguous()  # (E, G, N)
        zp = getattr(self, "weight_zero_point", None)
        if zp is None:
            self._zeros_op = None
        else:
            self._zeros_op = _method.apply_ct_sign(zp.contiguous(), conv).transpose(1, 2).contiguous()
            del self.weight_zero_point
        del self.weight_packed, self.weight_scale


class _GroupedMxFp4Experts:
    """MXFP4 experts: weight_packed (E, N, K/2) uint8 (two E2M1 nibbles per byte, low nibble =
    lower K), weight_scale (E, N, K/32) uint8 E8M0. After post_load: _w_op W4 tiles (e2m1 codes
    verbatim), _scales_op (E, K/32, N) E8M0 bytes, group-major."""

    def __init__(self, num_experts: int, out_features: int, in_features: int, quant):
        g = quant.group_size
        N, K = out_features, in_features
        assert K % 2 == 0 and K % g == 0 and N % 8 == 0, f"grouped MXFP4 needs K%2==0,K%{g}==0,N%8==0; got N={N},K={K}"
        self.weight_packed = torch.empty((num_experts, N, K // 2), dtype=torch.uint8)
        self.weight_scale = torch.empty((num_experts, N, K // g), dtype=torch.uint8)
        self._quant = quant
        self._num_experts = num_experts

    def forward(self, *args, **kwargs):
        raise RuntimeError(f"{type(self).__name__} holds weights; call kernels.w4a8_moe instead")

    def post_load(self) -> None:
        mxfp4 = importlib.import_module(f"{_pkg}.quant.mxfp4")
        conv = mxfp4.convert_mxfp4_moe_e8m0(self.weight_packed, self.weight_scale)
        self._scale_info = conv["scale_info"]
        self._w_op = _finish(conv["w_packed"], True)
        self._scales_op = conv["scales"].transpose(1, 2).contiguous()  # (E, K/32, N)
        self._zeros_op = None
        del self.weight_packed, self.weight_scale


class _GroupedNvFp4Experts:
    """NVFP4 experts (python/minisgl/layers/moe.py:346-407): weight_packed (E, N, K/2) uint8,
    weight_scale (E, N, K/16) float8_e4m3fn block scales (byte-verbatim), weight_global (E, N) f32
    per-output-channel multipliers (direction-normalised by the loader). After post_load: _w_op W4
    tiles, _scales_op (E, K/16, N) e4m3 group-major, _zeros_op the (E, N) globals' f32 bits as int32
    (the zeros slot of the grouped kernels)."""

    def __init__(self, num_experts: int, out_features: int, in_features: int, quant):
        N, K = out_features, in_features
        assert quant.group_size == 16, f"NVFP4 blocks are 16 elements; got group_size={quant.group_size}"
        assert K % 32 == 0 and N % 16 == 0, f"grouped NVFP4 needs K%32==0,N%16==0; got N={N},K={K}"
        self.weight_packed = torch.empty((num_experts, N, K // 2), dtype=torch.uint8)
        self.weight_scale = torch.empty((num_experts, N, K // 16), dtype=torch.float8_e4m3fn)
        self.weight_global = torch.empty((num_experts, N), dtype=torch.float32)
        self._quant = quant
        self._num_experts = num_experts

    def forward(self, *args, **kwargs):
        raise RuntimeError(f"{type(self).__name__} holds weights; call kernels.w4a8_moe instead")

    def post_load(self) -> None:
        nvfp4 = importlib.import_module(f"{_pkg}.quant.nvfp4")
        conv = nvfp4.convert_nvfp4_moe(self.weight_packed, self.weight_scale)
        self._w_op = _finish(conv["w_packed"], True)
        self._scales_op = conv["scales"].transpose(1, 2).contiguous()  # (E, K/16, N)
        # a view, never .to(int32): the value conversion would truncate every global to 0
        self._zeros_op = self.weight_global.to(torch.float32).contiguous().view(torch.int32)
        del self.weight_packed, self.weight_scale, self.weight_global


def _moe_w4a16() -> bool:
    """The W4A16 expert arm (unquantized activations), opt-in through MINISGL_MOE_W4A16 as in the
    reference (python/minisgl/layers/moe.py:649-670, 745-760, 816-873)."""
    return kernels.MOE_W4A16 != "0"


# Widest forward the NVFP4 experts serve through the W4A16 arm (python/minisgl/layers/moe.py:809-813);
# above it they stay W4A8 and the split is logged once.
_NVFP4_A16_DECODE_MAX = 2
_log = logging.getLogger("w4a8.nvfp4-moe")


def _w4a16_experts(quant, w13, w2, x, topk_weights, topk_ids, router_logits, top_k, renormalize, e2m1):
    """kernels.w4a16_moe over an int4 or MXFP4 expert pair (python/minisgl/layers/moe.py:663-670,
    752-760)."""
    inter = w13._scales_op.shape[2] // 2  # (E, G, 2*inter) group-major
    return kernels.w4a16_moe(x, w13._w_op, w13._scales_op, getattr(w13, "_zeros_op", None), w2._w_op, w2._scales_op,
                             getattr(w2, "_zeros_op", None), x.shape[1], inter, quant.group_size,
                             topk_weights=topk_weights, topk_ids=topk_ids, router_logits=router_logits, top_k=top_k,
                             renormalize=renormalize, weight_is_e2m1=e2m1)


class MoEQuantMethod:
    """How a MoE expert pair (w13 gate|up, w2 down) allocates its weights and runs its grouped GEMMs
    (python/minisgl/layers/moe.py:520-580)."""

    cache_plane_attrs: tuple = ()
    supports_ep: bool = False
    needs_precomputed_route: bool = False
    supports_producer_actquant: bool = False

    @classmethod
    def plane(cls, container):
        """This method's (w, scales, zeros) triple for one expert container."""
        return tuple(getattr(container, a) if a else None for a in cls.cache_plane_attrs)

    def create_experts(self, num_experts: int, out_features: int, in_features: int):
        raise NotImplementedError

    def apply(self, w13, w2, hidden_states, *, router_logits, topk_weights, topk_ids, top_k: int,
              renormalize: bool, activation: str, apply_router_weight_on_input: bool, x_fp8=None, act_scales=None):
        raise NotImplementedError

    def ep_local(self, w13, w2, g_hidden, local_weights, local_ids, *, top_k: int, renormalize: bool,
                 activation: str = "silu"):
        raise NotImplementedError(f"{type(self).__name__} does not support expert parallelism")


# gated activations the w4a8_moe family serves (python/minisgl/layers/moe.py:583-587): "gelu" is HF
# gelu_pytorch_tanh (Gemma4's routed experts), on the unfused gemm1 + gated tanh-GELU path
_W4A8_ACTIVATIONS = ("silu", "gelu")


def _check_activation(scheme: str, activation: str, allowed=_W4A8_ACTIVATIONS) -> None:
    if activation not in allowed:
        raise NotImplementedError(f"MoE {scheme} path supports activation {'|'.join(allowed)}; got {activation!r}")


def _reject_w4a16_activation(activation: str) -> None:
    # the W4A16 expert arm's tail is silu only: a gelu model reaching it would get well-formed wrong
    # numbers, so it is refused loudly (python/minisgl/layers/moe.py:678-690)
    if activation != "silu":
        raise NotImplementedError(f"MoE W4A16 (MINISGL_MOE_W4A16=1) is silu-only; got activation {activation!r}. "
                                  "Unset MINISGL_MOE_W4A16 to serve this model through the W4A8 path.")


class _W4A8MoEMethod(MoEQuantMethod):
    """int4 grouped experts (GPTQ, AWQ, compressed-tensors int4) through kernels.w4a8_moe."""

    supports_ep = True
    supports_producer_actquant = True
    cache_plane_attrs = ("_w_op", "_scales_op", "_zeros_op")

    def __init__(self, quant):
        self._quant = quant
        if quant.is_gptq:
            self._cls = _GroupedGPTQExperts
        elif quant.is_awq:
            self._cls = _GroupedAWQExperts
        elif quant.is_compressed_tensors:
            self._cls = _GroupedCompressedTensorsExperts
        else:
            raise AssertionError(f"W4A8 MoE unsupported quant method: {quant.method}")

    def create_experts(self, num_experts, out_features, in_features):
        return self._cls(num_experts, out_features, in_features, self._quant)

    def apply(self, w13, w2, hidden_states, *, router_logits, topk_weights, topk_ids, top_k, renormalize,
              activation, apply_router_weight_on_input, x_fp8=None, act_scales=None):
        _check_activation("W4A8", activation)
        assert not apply_router_weight_on_input, "MoE W4A8 path has no router-weight-on-input"
        if _moe_w4a16():
            _reject_w4a16_activation(activation)
            # fp16 activations, never quantized: a producer's fp8 pair has nothing to feed and is dropped
            return _w4a16_experts(self._quant, w13, w2, hidden_states, topk_weights, topk_ids, router_logits, top_k,
                                  renormalize, False)
        return kernels.w4a8_moe(hidden_states, w13._w_op, w13._scales_op, w13._zeros_op,
                                w2._w_op, w2._scales_op, w2._zeros_op, router_logits, top_k, renormalize,
                                topk_weights=topk_weights, topk_ids=topk_ids, activation=activation,
                                x_fp8=x_fp8, act_scales=act_scales)

    def ep_local(self, w13, w2, g_hidden, local_weights, local_ids, *, top_k, renormalize, activation="silu"):
        _check_activation("W4A8", activation)
        if _moe_w4a16():
            _reject_w4a16_activation(activation)
            return _w4a16_experts(self._quant, w13, w2, g_hidden, local_weights, local_ids, None, top_k, renormalize,
                                  False)
        return kernels.w4a8_moe(g_hidden, w13._w_op, w13._scales_op, w13._zeros_op,
                                w2._w_op, w2._scales_op, w2._zeros_op, None, top_k, renormalize,
                                topk_weights=local_weights, topk_ids=local_ids, activation=activation)


class _MxFp4MoEMethod(MoEQuantMethod):
    """MXFP4 grouped experts through kernels.w4a8_moe with weight_is_e2m1=True."""

    supports_ep = True
    supports_producer_actquant = True
    cache_plane_attrs = ("_w_op", "_scales_op", None)

    def __init__(self, quant):
        self._quant = quant

    def create_experts(self, num_experts, out_features, in_features):
        return _GroupedMxFp4Experts(num_experts, out_features, in_features, self._quant)

    def apply(self, w13, w2, hidden_states, *, router_logits, topk_weights, topk_ids, top_k, renormalize,
              activation, apply_router_weight_on_input, x_fp8=None, act_scales=None):
        _check_activation("MXFP4", activation)
        assert not apply_router_weight_on_input, "MoE MXFP4 path has no router-weight-on-input"
        if _moe_w4a16():
            _reject_w4a16_activation(activation)
            return _w4a16_experts(self._quant, w13, w2, hidden_states, topk_weights, topk_ids, router_logits, top_k,
                                  renormalize, True)
        return kernels.w4a8_moe(hidden_states, w13._w_op, w13._scales_op, None, w2._w_op, w2._scales_op, None,
                                router_logits, top_k, renormalize, topk_weights=topk_weights, topk_ids=topk_ids,
                                weight_is_e2m1=True, activation=activation, x_fp8=x_fp8, act_scales=act_scales)

    def ep_local(self, w13, w2, g_hidden, local_weights, local_ids, *, top_k, renormalize, activation="silu"):
        _check_activation("MXFP4", activation)
        if _moe_w4a16():
            _reject_w4a16_activation(activation)
            return _w4a16_experts(self._quant, w13, w2, g_hidden, local_weights, local_ids, None, top_k, renormalize,
                                  True)
        return kernels.w4a8_moe(g_hidden, w13._w_op, w13._scales_op, None, w2._w_op, w2._scales_op, None,
                                None, top_k, renormalize, topk_weights=local_weights, topk_ids=local_ids,
                                weight_is_e2m1=True, activation=activation)


class _NvFp4MoEMethod(MoEQuantMethod):
    """NVFP4 grouped experts through kernels.w4a8_moe: e2m1 codes, e4m3 block-16 scales and the
    (E, N) globals in the zeros slot (python/minisgl/layers/moe.py:785-883)."""

    supports_ep = True
    supports_producer_actquant = True
    cache_plane_attrs = ("_w_op", "_scales_op", "_zeros_op")

    def __init__(self, quant):
        self._quant = quant
        self._w4a16_split_logged = False

    def create_experts(self, num_experts, out_features, in_features):
        return _GroupedNvFp4Experts(num_experts, out_features, in_features, self._quant)

    def apply(self, w13, w2, hidden_states, *, router_logits, topk_weights, topk_ids, top_k, renormalize,
              activation, apply_router_weight_on_input, x_fp8=None, act_scales=None):
        _check_activation("NVFP4", activation)
        assert not apply_router_weight_on_input, "MoE NVFP4 path has no router-weight-on-input"
        if _moe_w4a16() and hidden_states.shape[0] <= _NVFP4_A16_DECODE_MAX:
            _reject_w4a16_activation(activation)
            return kernels.w4a16_moe_decode(hidden_states, *self.plane(w13), *self.plane(w2), hidden_states.shape[1],
                                            topk_weights=topk_weights, topk_ids=topk_ids, router_logits=router_logits,
                                            top_k=top_k, renormalize=renormalize)
        if _moe_w4a16() and not self._w4a16_split_logged:
            self._w4a16_split_logged = True
            _log.warning("MoE W4A16 on NVFP4 serves forwards of up to %d tokens; this one has %d and runs W4A8, so "
                         "activation precision splits by batch size", _NVFP4_A16_DECODE_MAX, hidden_states.shape[0])
        return kernels.w4a8_moe(hidden_states, w13._w_op, w13._scales_op, w13._zeros_op, w2._w_op, w2._scales_op,
                                w2._zeros_op, router_logits, top_k, renormalize, topk_weights=topk_weights,
                                topk_ids=topk_ids, weight_is_e2m1=True, activation=activation, x_fp8=x_fp8,
                                act_scales=act_scales)

    def ep_local(self, w13, w2, g_hidden, local_weights, local_ids, *, top_k, renormalize, activation="silu"):
        _check_activation("NVFP4", activation)
        return kernels.w4a8_moe(g_hidden, w13._w_op, w13._scales_op, w13._zeros_op, w2._w_op, w2._scales_op,
                                w2._zeros_op, None, top_k, renormalize, topk_weights=local_weights,
                                topk_ids=local_ids, weight_is_e2m1=True, activation=activation)


def create_moe_quant_method(quant, *, fp8_experts: bool = False) -> MoEQuantMethod:
    """Pick the expert method from the declared scheme (python/minisgl/layers/moe.py:971-1005):
    NVFP4 -> _NvFp4MoEMethod, MXFP4 -> _MxFp4MoEMethod, int4 AWQ/GPTQ/compressed-tensors ->
    _W4A8MoEMethod. Unquantized and fp8 experts are other paths and raise NotImplementedError here."""
    if fp8_experts or (quant is not None and quant.is_fp8_w8a8):
        raise NotImplementedError("fp8 W8A8 experts are not served by this W4A8 path")
    if quant is None:
        raise NotImplementedError("unquantized experts are not served by this W4A8 path")
    if quant.is_nvfp4:
        return _NvFp4MoEMethod(quant)
    if quant.weight_is_e2m1:
        return _MxFp4MoEMethod(quant)
    if quant.is_int4:
        return _W4A8MoEMethod(quant)
    raise AssertionError(f"MoE: unsupported declared quant scheme (method={quant.method}, bits={quant.bits}, "
                         f"weight_type={quant.weight_type})")
