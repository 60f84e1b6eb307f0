"""W4A8 kernel provider: the reference's ``minisgl.quant.kernels`` operator API on MI355X kernels.

Same names, argument meaning and refusal behaviour as python/minisgl/quant/kernels.py of the
reference for the W4A8 path: ``awq_to_op_layout`` / ``gptq_to_op_layout`` (:255-346),
``_moe_block_m`` (:355-420), ``_route_align`` (:423-447), ``_check_moe_scale_pair`` (:484-559),
``w4a8_moe`` (:562-882), ``_pick_dense_kernel`` (:1456-1632), ``w4a8_linear`` (:1686-1734),
``w4a8_linear_silu`` (:1737-1753). Underneath, every op calls libw4a8_mi355x.so through ctypes on
the current torch stream; outputs and workspaces are allocated here with torch, never in C.

Weights: the ops accept the reference's op layout (int32 ``(N, K/8)``, ``(E, N, K/8)`` for MoE) and
also the W4 tile layout (uint8 ``(N/16, ceil(K/128), 1024)``, ``(E, N/16, ceil(K/128), 1024)``)
that :func:`repack_w4` produces once at load. An op-layout weight is repacked on every call
(correct, and visible in the dispatch ledger as ``+repack``); the load path
(``method.W4A8LinearMethod``, the MoE containers) stores tiles so the serving call never repacks.
"""
from __future__ import annotations

import os

import torch

from .. import _abi
from .._hip_engage import engaged

# AWQ "gemm" reverse pack order: undoes the [0,2,4,6,1,3,5,7] channel interleave of AWQ packing
# (python/minisgl/quant/kernels.py:22).
_REVERSE_AWQ_PACK_ORDER = [0, 4, 1, 5, 2, 6, 3, 7]

# Decode band: the skinny-M kernel serves up to 16 rows (python/minisgl/quant/kernels.py:1663-1673
# sets the same ceiling for both weight formats) and consumes K in 32-element fragments.
_W4A8_GEMV_MAX_INT4 = 16
_W4A8_GEMV_MAX_E2M1 = 16
_W4A8_GEMV_K_MULTIPLE = 32

# The W4A16 arm (unquantized activations) of the linear methods is opt-in, read once at import
# (python/minisgl/quant/kernels.py MOE_W4A16 / MINISGL_MOE_W4A16).
MOE_W4A16 = os.environ.get("MINISGL_MOE_W4A16", "0")

# MoE gemm1 GEMV crossover and tile heights (python/minisgl/quant/kernels.py:130-131, 349-353).
_MOE_GEMM1_GEMV_MAX = 32
_MOE_WMMA_DIM = 16
_MOE_BLOCK_M_CHOICES = (16, 32, 64, 128)
# routed rows per expert up to which w4a8_moe runs the skinny grouped GEMV (block_m 16)
_MOE_SKINNY_MAX_ROWS = 32
# and 64-row MFMA tiles up to this many, 128-row tiles above
_MOE_MID_MAX_ROWS = 44
# gemm2 + top-k combine as one launch on the decode arm (python/minisgl/quant/kernels.py:831-850)
# up to _MOE_G2C_MAX_TOKENS tokens; MINISGL_MOE_G2FUSE=0 keeps the unfused path (requant, gemm2
# into (P, H) f32, combine), which gives the same bits. The fused kernel reads each routed expert's
# weights once per token where the grouped gemm2 reads them once per expert; measured on MI355X at
# configs[4] (whole w4a8_moe call, fused / unfused, us): T=1 25.2/29.5, 2 28.7/33.8, 4 34.0/39.0,
# 8 47.6/50.3, 12 60.7/59.9, 16 75.4/68.9 at first; with the fused kernel's tile loads all issued
# before their first use, T=10 49.8/55.3, 12 57.0/62.7, 14 62.8/67.6, 16 66.6/69.4 -- so up to 16.
_MOE_G2FUSE = os.environ.get("MINISGL_MOE_G2FUSE", "1") != "0"
_MOE_G2C_MAX_TOKENS = 16
# route, slots, the per-token quant of x and gemm1 as one launch for the calls that give every slot
# a block (w4a8_moe_route_gemm1); MINISGL_MOE_ROUTED=0 keeps the route + slots launch and gemm1,
# which give the same bits
_MOE_ROUTED = os.environ.get("MINISGL_MOE_ROUTED", "1") != "0"


# --------------------------------------------------------------------------------------------
# layout conversion (load time)
# --------------------------------------------------------------------------------------------
def _pack_along_last(vals: torch.Tensor, bits: int) -> torch.Tensor:
    """(..., L) small ints -> (..., L/pf) int32, element j of each group of pf in nibble j."""
    pf = 32 // bits
    mask = (1 << bits) - 1
    *lead, L = vals.shape
    v = (vals.to(torch.int64) & mask).reshape(*lead, L // pf, pf)
    shifts = torch.arange(0, 32, bits, dtype=torch.int64, device=vals.device)
    words = (v << shifts).sum(dim=-1)
    return (words & 0xFFFFFFFF).to(torch.int32)


def _unpack_along_last(words: torch.Tensor, bits: int) -> torch.Tensor:
    """(..., W) int32 -> (..., W*pf) int32 nibbles, nibble j of a word first-to-last."""
    pf = 32 // bits
    mask = (1 << bits) - 1
    shifts = torch.arange(0, 32, bits, dtype=torch.int32, device=words.device)
    u = (words.unsqueeze(-1) >> shifts) & mask
    return u.reshape(*words.shape[:-1], words.shape[-1] * pf)


def awq_to_op_layout(
    qweight: torch.Tensor,  # (K, N//pf) int32, AWQ-packed along the output dim, interleaved
    scales: torch.Tensor,  # (K//group, N) fp16
    qzeros: torch.Tensor | None,  # (K//group, N//pf) int32 AWQ-packed, or None (symmetric)
    *,
    bits: int = 4,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """One dense AWQ matrix -> op layout (w_packed (N, K/8) i32, scales (K/g, N) f16, zeros
    (K/g, N/8) i32 | None). Restates python/minisgl/quant/kernels.py:255-299: undo the AWQ column
    interleave, transpose to (N, K), repack 8 codes per int32 along K; zeros keep 8 channels per
    int32 along N in natural order; scales stay group-major."""
    assert bits == 4, "W4A8 path is 4-bit"
    K, Np = qweight.shape
    rev = torch.tensor(_REVERSE_AWQ_PACK_ORDER, dtype=torch.long, device=qweight.device)
    u = _unpack_along_last(qweight, bits).reshape(K, Np, 8)[:, :, rev].reshape(K, Np * 8)  # (K, N)
    w_packed = _pack_along_last(u.t().contiguous(), bits)  # (N, K/8)
    scales_op = scales.contiguous().to(torch.float16)
    zeros_op = None
    if qzeros is not None:
        G = qzeros.shape[0]
        uz = _unpack_along_last(qzeros, bits).reshape(G, Np, 8)[:, :, rev].reshape(G, Np * 8)
        zeros_op = _pack_along_last(uz, bits)
    return w_packed, scales_op, zeros_op


def gptq_to_op_layout(
    qweight: torch.Tensor,  # (K//pf, N) int32, packed along K, natural nibble order
    scales: torch.Tensor,  # (K//group, N) fp16
    qzeros: torch.Tensor | None,  # (K//group, N//pf) int32; stored zero + 1 is the zero point
    *,
    bits: int = 4,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One dense GPTQ matrix -> op layout. Restates python/minisgl/quant/kernels.py:302-346:
    unpack along K to (K, N), transpose, repack along K; zeros unpacked along N with AutoGPTQ's +1
    folded in (symmetric checkpoints store 7 -> zero 8), asserted to fit 4 bits."""
    assert bits == 4, "W4A8 path is 4-bit"
    assert qzeros is not None, "GPTQ always ships qzeros"
    Kp, N = qweight.shape
    K = Kp * 8
    u = _unpack_along_last(qweight.t().contiguous(), bits)  # (N, K): word kp nibble j -> k = 8kp + j
    w_packed = _pack_along_last(u, bits)
    scales_op = scales.contiguous().to(torch.float16)
    G = qzeros.shape[0]
    uz = _unpack_along_last(qzeros, bits).reshape(G, N) + 1
    assert int(uz.max()) <= 15, f"GPTQ zero+1 overflows 4b (max={int(uz.max())})"
    zeros_op = _pack_along_last(uz, bits)
    assert w_packed.shape == (N, K // 8)
    return w_packed, scales_op, zeros_op


def tile_shape(n: int, k: int) -> tuple[int, int, int]:
    return (n // 16, (k + 127) // 128, 1024)


def repack_w4(w_packed: torch.Tensor, weight_is_e2m1: bool = False) -> torch.Tensor:
    """Op layout -> W4 tile layout on the weight's device (one HIP launch).

    (N, K/8) int32 -> (N/16, ceil(K/128), 1024) uint8; (E, N, K/8) -> (E, N/16, ceil(K/128), 1024).
    """
    if w_packed.dtype != torch.int32 or w_packed.dim() not in (2, 3):
        raise TypeError(f"repack_w4: expected an int32 (N, K/8) or (E, N, K/8) tensor, got "
                        f"{w_packed.dtype} {tuple(w_packed.shape)}")
    if not w_packed.is_cuda:
        raise RuntimeError("repack_w4: the weight must be on the GPU (the repack is a HIP kernel)")
    lead = w_packed.shape[:-2]
    N, K = w_packed.shape[-2], w_packed.shape[-1] * 8
    rows = N * (w_packed.shape[0] if w_packed.dim() == 3 else 1)
    if N % 16:
        raise ValueError(f"repack_w4: N={N} must be a multiple of 16")
    out = torch.empty((*lead, *tile_shape(N, K)), dtype=torch.uint8, device=w_packed.device)
    lib = _abi.load()
    _abi.check(
        lib.w4a8_repack_weights(_abi.ptr(w_packed.contiguous()), rows, K,
                                _abi.W_E2M1 if weight_is_e2m1 else _abi.W_INT4, _abi.ptr(out),
                                _abi.stream_of(w_packed)),
        "repack_w4",
    )
    return out


def _as_tiles(w: torch.Tensor, k: int, weight_is_e2m1: bool, expect_dim: int, what: str) -> torch.Tensor:
    """Accept op layout (repacked now) or tiles; return tiles."""
    if w.dtype == torch.uint8 and w.dim() == expect_dim + 1 and w.shape[-1] == 1024:
        if w.shape[-2] != (k + 127) // 128:
            raise ValueError(f"{what}: tile tensor {tuple(w.shape)} does not match K={k}")
        return w
    if w.dtype == torch.int32 and w.dim() == expect_dim:
        if w.shape[-1] * 8 != k:
            raise ValueError(f"{what}: w_packed {tuple(w.shape)} does not match K={k}")
        return repack_w4(w, weight_is_e2m1)
    raise TypeError(f"{what}: weight must be op-layout int32 {'(E, N, K/8)' if expect_dim == 3 else '(N, K/8)'} "
                    f"or W4 tiles, got {w.dtype} {tuple(w.shape)}")


def _n_of(w: torch.Tensor) -> int:
    return w.shape[-3] * 16 if w.dtype == torch.uint8 else w.shape[-2]


# --------------------------------------------------------------------------------------------
# activation quant
# --------------------------------------------------------------------------------------------
def act_quant(x: torch.Tensor, row_count: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token fp8-e4m3 quant: returns (x_fp8 (M, K) uint8 e4m3fn codes, act_scales (M,) f32),
    the pair the reference's producer emits (python/minisgl/layers/norm.py:27-46) and its
    in-op pre-kernel computes (python/minisgl/quant/kernels.py:1703-1712)."""
    if x.dim() != 2 or x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"act_quant: x must be a 2-D bf16/fp16 tensor, got {x.dtype} {tuple(x.shape)}")
    x = x.contiguous()
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.uint8, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    lib = _abi.load()
    _abi.check(lib.w4a8_act_quant(_abi.ptr(x), _abi.dtype_code(x.dtype), M, K, K, _abi.ptr(q), K, _abi.ptr(s),
                                  _abi.ptr(row_count), _abi.stream_of(x)), "act_quant")
    return q, s


def _fp8_bytes(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t


# --------------------------------------------------------------------------------------------
# dense
# --------------------------------------------------------------------------------------------
_PREFILL_NAMES = ("wmma_tiled_tuned", "mfma_prefill")
_IN_PROLOGUE_NAMES = ("prefill_wmma", "prefill_wmma_ashuffle")


def _pick_dense_kernel(m: int, weight_is_e2m1: bool = False, group_size: int = 128,
                       k: int | None = None, n: int | None = None) -> str:
    """Per-M arm choice, same rule as python/minisgl/quant/kernels.py:1456-1632: the streaming
    decode kernel for M <= 16 when K is a multiple of 32, the MFMA tiled GEMM otherwise.
    ``MINISGL_FORCE_TILED_LINEARS=1`` forces the tiled arm at every M."""
    if os.environ.get("MINISGL_FORCE_TILED_LINEARS") == "1":
        return "wmma_tiled_tuned"
    gemv_max = _W4A8_GEMV_MAX_E2M1 if weight_is_e2m1 else _W4A8_GEMV_MAX_INT4
    if m <= gemv_max and (k is None or k % _W4A8_GEMV_K_MULTIPLE == 0):
        return "decode_gemv"
    return "wmma_tiled_tuned"


def _scale_fmt(scales: torch.Tensor, weight_is_e2m1: bool, what: str, has_zeros: bool = False) -> int:
    """The scale policy from the scales dtype plus the zeros slot (python/minisgl/quant/kernels.py:
    1137-1146, 518-559): fp16 -> folded group scales; uint8 without zeros -> MXFP4 E8M0; e4m3, or
    uint8 with the zeros slot populated -> NVFP4 block scales with the per-channel f32 global."""
    if scales.dtype == torch.float16:
        return _abi.SCALE_F16
    if scales.dtype in (torch.uint8, torch.float8_e4m3fn):
        if not weight_is_e2m1:
            raise TypeError(f"{what}: one-byte (E8M0 / e4m3) scales are only valid for e2m1 weights")
        if scales.dtype == torch.float8_e4m3fn or has_zeros:
            return _abi.SCALE_E4M3
        return _abi.SCALE_E8M0
    raise TypeError(f"{what}: scales must be fp16 (group scales), uint8 (E8M0) or float8_e4m3fn/uint8 with the "
                    f"NVFP4 global (e4m3 block scales), got {scales.dtype}")


def _nvfp4_global(w_zeros: torch.Tensor | None, N: int, what: str) -> torch.Tensor:
    """The NVFP4 per-output-channel f32 global multiplier, as the int32 bit pattern the zeros slot
    carries. A `.to(torch.int32)` of the floats instead of a view would truncate them, so only f32
    (viewed here) or an int32 bit pattern are accepted."""
    if w_zeros is None or w_zeros.numel() == 0:
        raise AssertionError(f"{what}: e4m3 block scales REQUIRE the per-output-channel f32 global in the "
                             f"zeros slot; the two-level scale is incomplete without it")
    if tuple(w_zeros.shape) != (N,) or w_zeros.dtype not in (torch.float32, torch.int32):
        raise AssertionError(f"{what}: the NVFP4 global must be an (N,)=({N},) f32 vector (or its int32 bit "
                             f"pattern), got {w_zeros.dtype} {tuple(w_zeros.shape)}")
    return w_zeros.contiguous().view(torch.int32)


def _check_producer_pair(x: torch.Tensor, x_fp8, act_scales, what: str):
    M, K = x.shape
    if (x_fp8 is None) != (act_scales is None):
        raise RuntimeError(f"{what}: x_fp8 and act_scales must be supplied TOGETHER (got only "
                           f"{'x_fp8' if x_fp8 is not None else 'act_scales'})")
    if x_fp8 is None:
        return None, None
    xq = _fp8_bytes(x_fp8)
    if xq.dtype != torch.uint8 or tuple(xq.shape) != (M, K) or not xq.is_contiguous():
        raise RuntimeError(f"{what}: x_fp8 must be a contiguous (M, K)=({M}, {K}) uint8/float8_e4m3fn tensor, "
                           f"got {x_fp8.dtype} {tuple(x_fp8.shape)}")
    if act_scales.dtype != torch.float32 or tuple(act_scales.shape) != (M,):
        raise RuntimeError(f"{what}: act_scales must be (M,)=({M},) float32, got {act_scales.dtype} "
                           f"{tuple(act_scales.shape)}")
    return xq, act_scales.contiguous()


def _dense_prep(x, w_packed, scales, w_zeros, group_size, weight_is_e2m1, what):
    """Shape/dtype checks shared by the dense arms; returns (M, K, N, sfmt, w_zeros, scales) with the
    zeros slot and the scales in the form the C ABI takes."""
    if x.dim() != 2 or x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"{what}: x must be 2-D bf16/fp16, got {x.dtype} {tuple(x.shape)}")
    M, K = x.shape
    N = _n_of(w_packed)
    G = K // group_size
    if K % group_size or tuple(scales.shape) != (G, N):
        raise AssertionError(f"{what}: scales must be GROUP-major (K//group, N)=({G}, {N}), got "
                             f"{tuple(scales.shape)}")
    has_zeros = w_zeros is not None and w_zeros.numel() > 0
    sfmt = _scale_fmt(scales, weight_is_e2m1, what, has_zeros)
    if sfmt == _abi.SCALE_E4M3:
        w_zeros = _nvfp4_global(w_zeros, N, what)
        scales = scales.view(torch.uint8)
    else:
        if weight_is_e2m1 and has_zeros:
            raise AssertionError(f"{what}: e2m1 weights are symmetric; w_zeros must be None")
        if not has_zeros:
            w_zeros = None
        if w_zeros is not None and (w_zeros.dtype != torch.int32 or tuple(w_zeros.shape) != (G, N // 8)):
            raise AssertionError(f"{what}: w_zeros must be (K//group, N/8)=({G}, {N // 8}) int32, got "
                                 f"{w_zeros.dtype} {tuple(w_zeros.shape)}")
    return M, K, N, sfmt, w_zeros, scales


def _dense(x, w_packed, scales, w_zeros, group_size, weight_is_e2m1, x_fp8, act_scales, silu, arm):
    what = "w4a8_linear_silu" if silu else "w4a8_linear"
    M, K, N, sfmt, w_zeros, scales = _dense_prep(x, w_packed, scales, w_zeros, group_size, weight_is_e2m1, what)
    xq, xs = _check_producer_pair(x, x_fp8, act_scales, what)
    tiles = _as_tiles(w_packed, K, weight_is_e2m1, 2, what)
    nout = N // 2 if silu else N
    out = torch.empty((M, nout), dtype=x.dtype, device=x.device)
    lib = _abi.load()
    zeros = _abi.ptr(w_zeros.contiguous() if w_zeros is not None else None)
    wfmt = _abi.W_E2M1 if weight_is_e2m1 else _abi.W_INT4
    sc = scales.contiguous()
    if xq is None:
        # the op quantizes x itself: in the decode kernel's prologue when the rows fit, else with
        # one act-quant launch into the workspace
        x = x.contiguous()
        ws_bytes = int(lib.w4a8_linear_workspace_bytes(M, K))
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=x.device)
        _abi.check(
            lib.w4a8_linear(_abi.ptr(x), _abi.dtype_code(x.dtype), M, K, K, _abi.ptr(tiles), N, _abi.ptr(sc),
                            sfmt, zeros, wfmt, group_size, _abi.ptr(out), _abi.dtype_code(x.dtype), nout, int(silu),
                            _abi.ptr(ws), ws_bytes, arm, _abi.stream_of(x)),
            what,
        )
    else:
        # prefill calls on wide weights may rewrite the codes in the GEMM's operand order first
        ws_bytes = int(lib.w4a8_gemm_workspace_bytes(M, N, K, arm))
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=x.device) if ws_bytes > 0 else None
        _abi.check(
            lib.w4a8_gemm(_abi.ptr(xq), K, _abi.ptr(xs), M, _abi.ptr(tiles), N, K, _abi.ptr(sc), sfmt, zeros, wfmt,
                          group_size, _abi.ptr(out), _abi.dtype_code(x.dtype), nout, int(silu), _abi.ptr(ws),
                          max(ws_bytes, 0), arm, _abi.stream_of(x)),
            what,
        )
    return out, tiles is not w_packed


def w4a8_linear(
    x: torch.Tensor,
    w_packed: torch.Tensor,  # (N, K/8) int32 op layout, or W4 tiles
    scales: torch.Tensor,  # (K/group, N) fp16 group-major, or uint8 E8M0 (e2m1 only)
    w_zeros: torch.Tensor | None,  # (K/group, N/8) int32 (asymmetric) or None (zero point 8)
    group_size: int,
    kernel: str | None = None,
    weight_is_e2m1: bool = False,
    x_fp8: torch.Tensor | None = None,  # producer-quantized activations (M, K) e4m3 codes
    act_scales: torch.Tensor | None = None,  # (M,) f32
) -> torch.Tensor:
    """Dense W4A8 GEMM (M, K) @ (N, K)^T -> (M, N) in x's dtype (python/minisgl/quant/
    kernels.py:1686-1734). Supplying the producer pair skips the op's own act-quant launch and is
    bit-identical to it. Names ``prefill_wmma``/``prefill_wmma_ashuffle`` are the reference's
    in-prologue-quant arms and refuse a pre-quantized pair loudly, as there."""
    N = _n_of(w_packed)
    K = x.shape[-1]
    if kernel is None:
        kernel = _pick_dense_kernel(x.shape[0], weight_is_e2m1, group_size, k=K, n=N)
    if kernel == "decode_gemv":
        arm = _abi.KERNEL_DECODE
    elif kernel in _PREFILL_NAMES or kernel in _IN_PROLOGUE_NAMES:
        if kernel in _IN_PROLOGUE_NAMES and x_fp8 is not None:
            raise RuntimeError(f"w4a8_linear: kernel={kernel} quantizes activations in-prologue and refuses a "
                               f"pre-quantized (x_fp8, act_scales) pair")
        arm = _abi.KERNEL_PREFILL
    else:
        raise ValueError(f"w4a8_linear: unknown kernel {kernel!r}")
    out, repacked = _dense(x, w_packed, scales, w_zeros, group_size, weight_is_e2m1, x_fp8, act_scales, False, arm)
    engaged(f"w4a8_mi355x.gemm({kernel}{'+e2m1' if weight_is_e2m1 else ''}"
            f"{'+prequant' if x_fp8 is not None else ''}{'+repack' if repacked else ''})")
    return out


def w4a8_linear_silu(
    x: torch.Tensor,
    w_packed: torch.Tensor,  # (2*inter, K/8) int32 [gate|up] op layout, or W4 tiles
    scales: torch.Tensor,
    w_zeros: torch.Tensor | None,
    group_size: int,
    weight_is_e2m1: bool = False,
) -> torch.Tensor:
    """Fused decode gate_up GEMV + silu_and_mul -> (M, inter) (python/minisgl/quant/
    kernels.py:1737-1753). Bit-exact to w4a8_linear(kernel="decode_gemv") followed by the
    round-silu-round-multiply replica of tools/w4a8_gemm_silu_parity.py:52-54."""
    if x.shape[0] > _W4A8_GEMV_MAX_INT4 or x.shape[1] % _W4A8_GEMV_K_MULTIPLE:
        raise AssertionError(f"w4a8_linear_silu: decode-only (M<=16, K%32==0), got {tuple(x.shape)}")
    out, repacked = _dense(x, w_packed, scales, w_zeros, group_size, weight_is_e2m1, None, None, True,
                           _abi.KERNEL_DECODE)
    engaged(f"w4a8_mi355x.gemm_silu({'e2m1' if weight_is_e2m1 else 'int4'}{'+repack' if repacked else ''})")
    return out


# --------------------------------------------------------------------------------------------
# MoE
# --------------------------------------------------------------------------------------------
def _w4a16(x, w_packed, scales, w_zeros, group_size, weight_is_e2m1, silu, what):
    M, K, N, sfmt, w_zeros, scales = _dense_prep(x, w_packed, scales, w_zeros, group_size, weight_is_e2m1, what)
    tiles = _as_tiles(w_packed, K, weight_is_e2m1, 2, what)
    if K % 8:
        raise AssertionError(f"{what}: K={K} must be a multiple of 8")
    kernel = _pick_dense_kernel(M, weight_is_e2m1, group_size, k=K, n=N)
    arm = _abi.KERNEL_DECODE if kernel == "decode_gemv" else _abi.KERNEL_PREFILL
    nout = N // 2 if silu else N
    x = x.contiguous()
    out = torch.empty((M, nout), dtype=x.dtype, device=x.device)
    lib = _abi.load()
    ws_bytes = int(lib.w4a16_linear_workspace_bytes(M, N, K, _abi.dtype_code(x.dtype)))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=x.device)
    zeros = _abi.ptr(w_zeros.contiguous() if w_zeros is not None else None)
    wfmt = _abi.W_E2M1 if weight_is_e2m1 else _abi.W_INT4
    _abi.check(
        lib.w4a16_linear(_abi.ptr(x), _abi.dtype_code(x.dtype), M, K, K, _abi.ptr(tiles), N,
                         _abi.ptr(scales.contiguous()), sfmt, zeros, wfmt, group_size, _abi.ptr(out), nout,
                         int(silu), _abi.ptr(ws), ws_bytes, arm, _abi.stream_of(x)),
        what,
    )
    return out, kernel


def w4a16_linear(
    x: torch.Tensor,  # (M, K) bf16/fp16 activations, never quantized
    w_packed: torch.Tensor,  # (N, K/8) int32 op layout, or W4 tiles (the same weights the W4A8 arms take)
    scales: torch.Tensor,  # (K/group, N) fp16 group-major, or uint8 E8M0 (e2m1 only)
    w_zeros: torch.Tensor | None,  # (K/group, N/8) int32 (asymmetric) or None
    group_size: int,
    N: int,
    weight_is_e2m1: bool = False,
) -> torch.Tensor:
    """Dense W4A16 GEMM (python/minisgl/quant/kernels.py:1125-1178): (M, K) @ (N, K)^T in x's dtype
    with the activations unquantized. The arm follows M as in the reference (decode GEMV up to 16
    tokens, the tiled GEMM above); both take the W4A8 weights as they are. The activations enter the
    fp8 MFMA kernels through an exact split into fp8 terms (two for bf16, three for fp16) whose f32
    partial results are summed per token before the one rounding to the output dtype."""
    if _n_of(w_packed) != N:
        raise AssertionError(f"w4a16_linear: N={N} does not match the weight's {_n_of(w_packed)} rows")
    out, kernel = _w4a16(x, w_packed, scales, w_zeros, group_size, weight_is_e2m1, False, "w4a16_linear")
    engaged(f"w4a8_mi355x.w4a16_{'gemv' if kernel == 'decode_gemv' else 'tiled'}"
            f"{'+e2m1' if weight_is_e2m1 else ''}")
    return out


def w4a16_linear_silu(
    x: torch.Tensor,
    w_packed: torch.Tensor,  # (2*inter, K/8) [gate | up]
    scales: torch.Tensor,
    w_zeros: torch.Tensor | None,
    group_size: int,
    weight_is_e2m1: bool = False,
) -> torch.Tensor:
    """Fused gate_up W4A16 + silu_and_mul -> (M, inter) (python/minisgl/quant/kernels.py:1756-1786):
    gate and up are the w4a16_linear outputs rounded to the dtype, then silu(gate) in f32, rounded,
    times up, rounded; bit-identical to w4a16_linear followed by that silu_mul."""
    out, kernel = _w4a16(x, w_packed, scales, w_zeros, group_size, weight_is_e2m1, True, "w4a16_linear_silu")
    engaged(f"w4a8_mi355x.w4a16_{'gemv' if kernel == 'decode_gemv' else 'tiled'}_silu"
            f"{'+e2m1' if weight_is_e2m1 else ''}")
    return out


def w4a16_act_split(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The activation side of the W4A16 arm: (T*M, K) uint8 e4m3 codes and (T*M,) f32 power-of-two
    scales with x[m] == sum_t scales[T*m+t] * e4m3(codes[T*m+t]) (T = 2 for bf16, 3 for fp16)."""
    if x.dim() != 2 or x.dtype not in (torch.bfloat16, torch.float16) or x.shape[1] % 8:
        raise TypeError(f"w4a16_act_split: x must be 2-D bf16/fp16 with K % 8 == 0, got {x.dtype} {tuple(x.shape)}")
    x = x.contiguous()
    M, K = x.shape
    T = 2 if x.dtype == torch.bfloat16 else 3
    q = torch.empty((T * M, K), dtype=torch.uint8, device=x.device)
    s = torch.empty((T * M,), dtype=torch.float32, device=x.device)
    lib = _abi.load()
    _abi.check(lib.w4a16_act_split(_abi.ptr(x), _abi.dtype_code(x.dtype), M, K, K, _abi.ptr(q), K, _abi.ptr(s),
                                   _abi.stream_of(x)), "w4a16_act_split")
    return q, s


def _moe_block_m(num_tokens: int, num_experts: int, top_k: int, flag_gemm1: bool | None = None) -> int:
    """Grouped-GEMM tile height from the workload (python/minisgl/quant/kernels.py:355-420): the
    largest of 16/32/64/128 not above the mean rows per expert; past the gemm1 GEMV crossover
    (M > 32) at least 64 when the fused-silu tiled arm can run. ``MINISGL_MOE_BLOCK_M`` forces it.
    Here block_m < 64 selects the skinny-M grouped kernel, block_m % 64 == 0 the MFMA tiled one."""
    forced = os.environ.get("MINISGL_MOE_BLOCK_M")
    if forced:
        bm = int(forced)
        assert bm in _MOE_BLOCK_M_CHOICES, f"MINISGL_MOE_BLOCK_M must be one of {_MOE_BLOCK_M_CHOICES}"
        return bm
    rows_per_expert = (num_tokens * top_k) / max(num_experts, 1)
    bm = _MOE_WMMA_DIM
    for choice in _MOE_BLOCK_M_CHOICES:
        if choice <= rows_per_expert:
            bm = choice
    if flag_gemm1 is None or num_tokens <= _MOE_GEMM1_GEMV_MAX:
        return bm
    if flag_gemm1:
        return max(bm, 64)
    wide = bm
    for choice in _MOE_BLOCK_M_CHOICES:
        if choice <= min(2 * rows_per_expert, 64):
            wide = choice
    return max(bm, wide)


def _moe_block_m_auto(num_tokens: int, num_experts: int, top_k: int) -> int:
    """The tile height w4a8_moe picks when the caller gives none, from MI355X measurements of these
    kernels at the configs[4] shape (E=128, top-8, H=2048, I=768), whole call, us:
    - the skinny grouped GEMV (16-row blocks) up to 32 routed rows per expert, where it streams
      each expert's weights once per 16 rows (T=256: 121, against 173 with 64-row tiles and 194
      with 128; T=512, 32 rows: 178 against 180 and 197);
    - 64-row MFMA tiles up to 44 rows (T=640, 40 rows: 177, against 205 with the GEMV and 192
      with 128-row tiles);
    - 128-row tiles above (T=768: 195 against 197 at 64; T=1024: 200 against 252; T=4096: 502
      against 738).
    The reference raises to 64 past 32 tokens because its own GEMV arm loses there
    (``_moe_block_m``, kept as written for callers and tests that want that rule).
    ``MINISGL_MOE_BLOCK_M`` still forces a value."""
    if os.environ.get("MINISGL_MOE_BLOCK_M"):
        return _moe_block_m(num_tokens, num_experts, top_k)
    rows_per_expert = (num_tokens * top_k) / max(num_experts, 1)
    if rows_per_expert <= _MOE_SKINNY_MAX_ROWS:
        return 16
    return 64 if rows_per_expert <= _MOE_MID_MAX_ROWS else 128


def _route_align(gating_output: torch.Tensor, top_k: int, renormalize: bool, num_experts: int,
                 block_size: int):
    """softmax + top-k + renormalize + align in one call (python/minisgl/quant/kernels.py:423-447).
    Returns (topk_weights f32, topk_ids i32, sorted_ids, expert_ids, num_tokens_post_pad)."""
    r = _route_align_quant(gating_output, top_k, renormalize, num_experts, block_size, None)
    return r[0], r[1], r[2], r[3], r[4]


def _route_align_quant(gating_output: torch.Tensor, top_k: int, renormalize: bool, num_experts: int,
                       block_size: int, x: torch.Tensor | None, slots: bool = False):
    """Route + align (+ per-token act quant of x when given) through w4a8_moe_route_align: one
    launch for up to 256 slots. Returns (tw, ids, sorted_ids, expert_ids, ntp, inv_pos, x_fp8,
    x_scales); the last two are None without x. slots: w4a8_moe_route_slots instead (one block per
    slot, no align; only the rows below ntp are written)."""
    engaged("w4a8_mi355x.moe_route_slots" if slots else "w4a8_mi355x.moe_route_align")
    g = gating_output.contiguous()
    if g.dim() != 2 or g.shape[1] != num_experts:
        raise AssertionError(f"moe route: gating_output must be (M, E={num_experts}), got {tuple(g.shape)}")
    T = g.shape[0]
    dev = g.device
    numel = T * top_k
    lib = _abi.load()
    P = int(lib.w4a8_moe_padded_capacity(numel, num_experts, block_size))
    # one block per slot needs a block per slot within the capacity, and no more slots than experts
    # (the grouped GEMMs size their grids for at most numel / block + min(E, numel) blocks)
    slots = slots and numel <= num_experts and numel * block_size <= P
    tw = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    ids = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    sorted_ids = torch.empty((P,), dtype=torch.int32, device=dev)
    expert_ids = torch.empty(((P + block_size - 1) // block_size,), dtype=torch.int32, device=dev)
    ntp = torch.empty((1,), dtype=torch.int32, device=dev)
    inv = torch.empty((max(numel, 1),), dtype=torch.int32, device=dev)
    xq = xs = None
    K = ldx = 0
    xdt = 0
    if x is not None:
        xc = x if x.stride(-1) == 1 else x.contiguous()
        K, ldx = xc.shape[1], xc.stride(0)
        xdt = _abi.dtype_code(xc.dtype)
        xq = torch.empty((T, K), dtype=torch.uint8, device=dev)
        xs = torch.empty((T,), dtype=torch.float32, device=dev)
        x = xc
    fn = lib.w4a8_moe_route_slots if slots else lib.w4a8_moe_route_align
    _abi.check(fn(_abi.ptr(g), _abi.dtype_code(g.dtype), T, num_experts, top_k, int(bool(renormalize)), block_size, P,
                  _abi.ptr(tw), _abi.ptr(ids), _abi.ptr(sorted_ids), _abi.ptr(expert_ids), _abi.ptr(ntp),
                  _abi.ptr(inv), _abi.ptr(x) if x is not None else None, xdt, K, ldx,
                  _abi.ptr(xq) if xq is not None else None, K, _abi.ptr(xs) if xs is not None else None,
                  _abi.stream_of(g)),
               "moe_route_slots" if slots else "moe_route_align")
    return tw, ids, sorted_ids, expert_ids, ntp, inv, xq, xs


def _route_gemm1(gating_output, top_k, renormalize, E, block_m, x, t13, N1, w13s, s13f, w13z, wfmt, group):
    """w4a8_moe_route_gemm1: route + one block per slot + gemm1 with the silu epilogue of a
    decode-sized batch in one launch, every gemm1 workgroup routing its slot's token itself.
    Returns (tw, ids, sorted_ids, expert_ids, ntp, inv_pos, gemm1 buffer), the same tensors and
    bits as w4a8_moe_route_slots followed by the grouped gemm1, or None where the library does not
    cover the call (formats, sizes); nothing is launched then."""
    g = gating_output.contiguous()
    if g.dim() != 2 or g.shape[1] != E:
        raise AssertionError(f"moe route: gating_output must be (M, E={E}), got {tuple(g.shape)}")
    xc = x if x.stride(-1) == 1 else x.contiguous()
    T, K = xc.shape
    numel = T * top_k
    lib = _abi.load()
    P = int(lib.w4a8_moe_padded_capacity(numel, E, block_m))
    if numel > E or numel * block_m > P:
        return None
    dev = g.device
    tw = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    ids = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    sorted_ids = torch.empty((P,), dtype=torch.int32, device=dev)
    expert_ids = torch.empty(((P + block_m - 1) // block_m,), dtype=torch.int32, device=dev)
    ntp = torch.empty((1,), dtype=torch.int32, device=dev)
    inv = torch.empty((max(numel, 1),), dtype=torch.int32, device=dev)
    buf2 = torch.empty((P, N1 // 2), dtype=xc.dtype, device=dev)
    rc = lib.w4a8_moe_route_gemm1(
        _abi.ptr(g), _abi.dtype_code(g.dtype), T, E, top_k, int(bool(renormalize)), _abi.ptr(xc),
        _abi.dtype_code(xc.dtype), xc.stride(0), block_m, P, _abi.ptr(t13), N1, K, _abi.ptr(w13s), s13f, _abi.ptr(w13z),
        wfmt, group, _abi.ptr(tw), _abi.ptr(ids), _abi.ptr(sorted_ids), _abi.ptr(expert_ids), _abi.ptr(ntp),
        _abi.ptr(inv), _abi.ptr(buf2), _abi.dtype_code(xc.dtype), N1 // 2, _abi.stream_of(xc))
    if rc == _abi.ERR_UNSUPPORTED:
        return None
    _abi.check(rc, "w4a8_moe route_gemm1")
    return tw, ids, sorted_ids, expert_ids, ntp, inv, buf2


def _moe_route(gating_output: torch.Tensor, top_k: int, renormalize: bool, num_experts: int):
    engaged("w4a8_mi355x.moe_route_align")
    g = gating_output.contiguous()
    if g.dim() != 2 or g.shape[1] != num_experts:
        raise AssertionError(f"moe route: gating_output must be (M, E={num_experts}), got {tuple(g.shape)}")
    T = g.shape[0]
    tw = torch.empty((T, top_k), dtype=torch.float32, device=g.device)
    ids = torch.empty((T, top_k), dtype=torch.int32, device=g.device)
    lib = _abi.load()
    _abi.check(lib.w4a8_moe_route(_abi.ptr(g), _abi.dtype_code(g.dtype), T, num_experts, top_k, int(bool(renormalize)),
                                  _abi.ptr(tw), _abi.ptr(ids), _abi.stream_of(g)), "moe_route")
    return tw, ids


def _moe_align(topk_ids: torch.Tensor, num_experts: int, block_size: int):
    ids = topk_ids.to(torch.int32).contiguous()
    numel = ids.numel()
    lib = _abi.load()
    P = int(lib.w4a8_moe_padded_capacity(numel, num_experts, block_size))
    dev = ids.device
    sorted_ids = torch.empty((P,), dtype=torch.int32, device=dev)
    expert_ids = torch.empty(((P + block_size - 1) // block_size,), dtype=torch.int32, device=dev)
    ntp = torch.empty((1,), dtype=torch.int32, device=dev)
    inv = torch.empty((max(numel, 1),), dtype=torch.int32, device=dev)
    _abi.check(lib.w4a8_moe_align(_abi.ptr(ids), numel, num_experts, block_size, P, _abi.ptr(sorted_ids),
                                  _abi.ptr(expert_ids), _abi.ptr(ntp), _abi.ptr(inv), _abi.stream_of(ids)),
               "moe_align")
    return sorted_ids, expert_ids, ntp, inv


def moe_align(topk_ids: torch.Tensor, num_experts: int, block_size: int):
    """moe_align_block_size (python/minisgl/moe/fused.py:120-176) -> (sorted_ids, expert_ids, ntp)."""
    engaged("w4a8_mi355x.moe_align")
    s, e, n, _ = _moe_align(topk_ids, num_experts, block_size)
    return s, e, n


def _check_moe_scale_pair(w: torch.Tensor, scales: torch.Tensor, zeros: "torch.Tensor | None", which: str) -> None:
    """The (scales dtype, zeros slot) pair must be one the grouped kernel dispatches
    (python/minisgl/quant/kernels.py:484-559): fp16 folded scales with optional (E, G, N/8) AWQ
    zeros; uint8 without zeros is MXFP4 E8M0. The NVFP4 two-level form (e4m3/uint8 block scale
    with an (E, N) f32-as-int32 global) is validated exactly as there and served by the e2m1
    kernels with 16-wide groups."""
    if scales.dtype == torch.float16:
        if zeros is not None and zeros.dim() != 3:
            raise AssertionError(
                f"w4a8_moe {which}: fp16 (folded) scales pair with AWQ packed zeros (E, G, N/8) int32, but got a "
                f"{zeros.dim()}-D {zeros.dtype} tensor {tuple(zeros.shape)}. A 2-D zeros tensor here is an NVFP4 "
                f"per-output-channel global handed to the fp16 policy, which would stride it as if it were (E, G, N/8)."
            )
        return
    if scales.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise AssertionError(
            f"w4a8_moe {which}: scales must be fp16 (folded per-group), float8_e4m3fn/uint8 (NVFP4 two-level block "
            f"scale) or uint8 with no zeros (MXFP4 E8M0); got {scales.dtype}"
        )
    E, N = w.shape[0], _n_of(w)
    if scales.dtype == torch.uint8 and zeros is None:
        return
    if zeros is None:
        raise AssertionError(
            f"w4a8_moe {which}: e4m3 block scales REQUIRE the per-output-channel f32 global in the zeros slot -- "
            f"the two-level scale is incomplete without it."
        )
    if zeros.dtype != torch.int32 or tuple(zeros.shape) != (E, N):
        raise AssertionError(
            f"w4a8_moe {which}: the NVFP4 global must be the (E, N)=({E}, {N}) f32 vector BITCAST to int32; got "
            f"{zeros.dtype} {tuple(zeros.shape)}. A `.to(torch.int32)` instead of `.view(torch.int32)` truncates "
            f"every global to 0."
        )


def _moe_gemm2_combine(buf2, topk_ids, tw, inv, T, top_k, bm, P, tiles, E, H, inter, scales, sfmt, zeros, wfmt,
                       group, out, row_dtype):
    """gemm2 (per-row requant of the gemm1 buffer in the prologue) + top-k weighted combine as one
    launch: fp8_wmma.mmq_fp8_moe_gemm2_gather_reduce (python/minisgl/quant/kernels.py:831-850);
    each slot's gemm2 row rounded to row_dtype first (float32: not rounded)."""
    lib = _abi.load()
    _abi.check(
        lib.w4a8_moe_gemm2_combine(_abi.ptr(buf2), _abi.dtype_code(buf2.dtype), buf2.stride(0), _abi.ptr(topk_ids),
                                   _abi.ptr(tw), _abi.ptr(inv), T, top_k, bm, P, _abi.ptr(tiles), E, H, inter,
                                   _abi.ptr(scales), sfmt, _abi.ptr(zeros), wfmt, group, _abi.ptr(out),
                                   _abi.dtype_code(out.dtype), out.stride(0), _abi.dtype_code(row_dtype),
                                   _abi.stream_of(buf2)),
        "w4a8_moe gemm2+combine",
    )


def _moe_gemm(a, lda, a_scales, a_by_token, sorted_ids, expert_ids, ntp, numel, top_k, bm, P, tiles, E, N, K,
              scales, sfmt, zeros, wfmt, group, out, out_dtype, ldo, silu, arm, what):
    lib = _abi.load()
    ws_bytes = int(lib.w4a8_moe_gemm_workspace_bytes(numel, E, bm, P, N, K, arm))
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=a.device) if ws_bytes > 0 else None
    _abi.check(
        lib.w4a8_moe_gemm(_abi.ptr(a), lda, _abi.ptr(a_scales), a_by_token, _abi.ptr(sorted_ids), _abi.ptr(expert_ids),
                          _abi.ptr(ntp), numel, top_k, bm, P, _abi.ptr(tiles), E, N, K, _abi.ptr(scales), sfmt,
                          _abi.ptr(zeros), wfmt, group, _abi.ptr(out), out_dtype, ldo, int(silu), _abi.ptr(ws),
                          ws_bytes, arm, _abi.stream_of(a)),
        what,
    )


def w4a8_moe(
    x: torch.Tensor,  # (M, K) activations
    w13: torch.Tensor,  # (E, 2*inter, K//8) i32 op layout (gate | up), or W4 tiles
    w13_scales: torch.Tensor,  # (E, K//g, 2*inter) group-major fp16, or uint8 E8M0 (e2m1)
    w13_zeros: torch.Tensor | None,  # (E, K//g, 2*inter/8) i32 AWQ zeros | None
    w2: torch.Tensor,  # (E, K, inter//8) i32 op layout, or W4 tiles
    w2_scales: torch.Tensor,  # (E, inter//g, K)
    w2_zeros: torch.Tensor | None,
    gating_output: torch.Tensor | None,  # (M, E); ignored when topk_ids/topk_weights are given
    top_k: int,
    renormalize: bool,
    *,
    topk_weights: torch.Tensor | None = None,
    topk_ids: torch.Tensor | None = None,
    kernel: str = "wmma",
    block_m: int | None = None,
    weight_is_e2m1: bool = False,
    activation: str = "silu",
    x_fp8: torch.Tensor | None = None,
    act_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """Grouped W4A8 MoE forward (python/minisgl/quant/kernels.py:562-882): route -> align ->
    gemm1 with fused silu(gate)*up (output in x's dtype) -> per-row act-quant of that buffer ->
    gemm2 -> top-k weighted combine in f32 -> x's dtype. Returns (M, K)."""
    return _moe_forward(x, w13, w13_scales, w13_zeros, w2, w2_scales, w2_zeros, gating_output, top_k, renormalize,
                        topk_weights=topk_weights, topk_ids=topk_ids, block_m=block_m, weight_is_e2m1=weight_is_e2m1,
                        activation=activation, x_fp8=x_fp8, act_scales=act_scales)["out"]


_MOE_SLOTS_MAX = int(os.environ.get("W4A8_MOE_SLOTS_MAX", "8"))


def _moe_forward(x, w13, w13_scales, w13_zeros, w2, w2_scales, w2_zeros, gating_output, top_k, renormalize, *,
                 topk_weights=None, topk_ids=None, block_m=None, weight_is_e2m1=False, activation="silu",
                 x_fp8=None, act_scales=None, y2_dtype=None) -> dict:
    """w4a8_moe's pipeline; returns the output and every intermediate (route, align, the (P, inter)
    gemm1 buffer) so each stage can be checked on its own. The gemm2 rows reach the combine as the
    reference hands them over: unrounded (f32) where it runs its fused decode gemm2 + gather-reduce
    (MINISGL_MOE_G2FUSE on, no NVFP4 two-level scales, M <= 32, block_m != 128:
    python/minisgl/quant/kernels.py:836-850), in x's dtype where it runs the unfused gemm2
    (kernels.py:852-882, tools/vhip_patches/moe_experts.py:874-880); this holds on both of this
    build's gemm2 paths ("round_y2" in the result). y2_dtype overrides the unfused path's row dtype
    (tests run it in f32 to compare with the fused kernel)."""
    M, K = x.shape
    E = w13.shape[0]
    _grp = (K // w13_scales.shape[1]) if w13_scales.dim() == 3 else -1
    assert _grp in (16, 32, 64, 128), (
        f"w4a8_moe: derived group_size={_grp} from K={K} and G={w13_scales.shape[1]}; scales must be GROUP-major "
        f"(E, K//group, N), got {tuple(w13_scales.shape)}"
    )
    _check_moe_scale_pair(w13, w13_scales, w13_zeros, "w13")
    _check_moe_scale_pair(w2, w2_scales, w2_zeros, "w2")
    assert activation in ("silu", "gelu"), (
        f"w4a8_moe supports activation 'silu' or 'gelu' (gelu_pytorch_tanh); got {activation!r}")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"w4a8_moe: x must be bf16/fp16, got {x.dtype}")
    N1 = _n_of(w13)
    inter = N1 // 2
    H2 = _n_of(w2)
    if H2 != K:
        raise AssertionError(f"w4a8_moe: w2 has {H2} output channels, expected hidden size {K}")
    _grp2 = inter // w2_scales.shape[1]
    if block_m is None:
        block_m = _moe_block_m_auto(M, E, top_k)

    if x_fp8 is not None:
        assert act_scales is not None, "w4a8_moe: x_fp8 and act_scales must be supplied together"
        assert tuple(x_fp8.shape) == (M, K) and tuple(act_scales.shape) == (M,), (
            f"w4a8_moe: producer pair must be (M,K)=({M},{K}) and (M,)=({M},); got {tuple(x_fp8.shape)} and "
            f"{tuple(act_scales.shape)}")
    elif act_scales is not None:
        raise AssertionError("w4a8_moe: act_scales given without x_fp8")

    wfmt = _abi.W_E2M1 if weight_is_e2m1 else _abi.W_INT4
    t13 = _as_tiles(w13, K, weight_is_e2m1, 3, "w4a8_moe w13")
    t2 = _as_tiles(w2, inter, weight_is_e2m1, 3, "w4a8_moe w2")
    s13f = _scale_fmt(w13_scales, weight_is_e2m1, "w4a8_moe w13", w13_zeros is not None)
    s2f = _scale_fmt(w2_scales, weight_is_e2m1, "w4a8_moe w2", w2_zeros is not None)
    if s13f == _abi.SCALE_E4M3:
        w13_scales = w13_scales.view(torch.uint8)
    if s2f == _abi.SCALE_E4M3:
        w2_scales = w2_scales.view(torch.uint8)
    w13s = w13_scales.contiguous()
    w13z = w13_zeros.contiguous() if w13_zeros is not None else None
    arm = _abi.KERNEL_DECODE if block_m < 64 else _abi.KERNEL_PREFILL
    arm_name = "gemv" if arm == _abi.KERNEL_DECODE else "mfma"
    e2 = "+e2m1" if weight_is_e2m1 else ""

    # Up to _MOE_SLOTS_MAX tokens on the decode arm: one block per slot instead of the align (one
    # token's experts are distinct, so the align would share no block either; a few tokens share
    # few, and a shared expert's weights are then streamed once per slot). configs[4], whole call,
    # align -> slots: T=1 23.9 -> 21.1 us, T=2 28.5 -> 25.6, T=4 34.3 -> 31.0, T=8 50.9 -> 47.8;
    # T=16 68.8 -> 79.0, so the align stays from there on
    slots = M <= _MOE_SLOTS_MAX and block_m < 64
    buf2 = None
    gelu = activation == "gelu"
    buf1 = None
    if topk_ids is None and x_fp8 is None and slots and _MOE_ROUTED and not gelu:
        # route, slots, the per-token quant of x and gemm1 in one launch (same bits as below)
        r = _route_gemm1(gating_output, top_k, renormalize, E, block_m, x, t13, N1, w13s, s13f, w13z, wfmt, _grp)
        if r is not None:
            topk_weights, topk_ids, sorted_ids, expert_ids, ntp, inv, buf2 = r
            engaged(f"w4a8_mi355x.moe_route_gemm1_silu(gemv{e2})")
    if buf2 is None:
        xq = xs = None
        if topk_ids is None:
            # route + align (or slots), and the per-token quant of x unless the producer supplied
            # it (one launch for small batches); the inverse positions (slot -> padded row) feed
            # the combine
            topk_weights, topk_ids, sorted_ids, expert_ids, ntp, inv, xq, xs = _route_align_quant(
                gating_output, top_k, renormalize, E, block_m, x if x_fp8 is None else None, slots=slots)
        else:
            assert topk_weights is not None, "topk_weights required when topk_ids is given"
            topk_weights = topk_weights.to(torch.float32).contiguous()
            topk_ids = topk_ids.to(torch.int32).contiguous()
            engaged("w4a8_mi355x.moe_align")
            sorted_ids, expert_ids, ntp, inv = _moe_align(topk_ids, E, block_m)
        if x_fp8 is not None:
            xq, xs = _fp8_bytes(x_fp8).contiguous(), act_scales.to(torch.float32).contiguous()
        elif xq is None:
            xq, xs = act_quant(x)
        P = sorted_ids.shape[0]
        buf2 = torch.empty((P, inter), dtype=x.dtype, device=x.device)
        pq = '+prequant' if x_fp8 is not None else ''
        if gelu:
            # HF gelu_pytorch_tanh experts: the unfused gemm1 ((P, 2*inter) in x's dtype), then the
            # gated tanh-GELU (python/minisgl/quant/kernels.py:768-783)
            buf1 = torch.empty((P, N1), dtype=x.dtype, device=x.device)
            engaged(f"w4a8_mi355x.moe_gemm1({arm_name}{e2}{pq})")
            _moe_gemm(xq, K, xs, 1, sorted_ids, expert_ids, ntp, topk_ids.numel(), top_k, block_m, P, t13, E, N1, K,
                      w13s, s13f, w13z, wfmt, _grp, buf1, _abi.dtype_code(x.dtype), N1, False, arm, "w4a8_moe gemm1")
            engaged("w4a8_mi355x.moe_gelu_tanh_mul")
            _abi.check(_abi.load().w4a8_moe_gelu_tanh_mul(_abi.ptr(buf1), _abi.dtype_code(x.dtype), N1, P, inter,
                                                          _abi.ptr(buf2), inter, _abi.ptr(ntp), _abi.stream_of(x)),
                       "w4a8_moe gelu_tanh_mul")
        else:
            engaged(f"w4a8_mi355x.moe_gemm1_silu({arm_name}{e2}{pq})")
            _moe_gemm(xq, K, xs, 1, sorted_ids, expert_ids, ntp, topk_ids.numel(), top_k, block_m, P, t13, E, N1, K,
                      w13s, s13f, w13z, wfmt, _grp, buf2, _abi.dtype_code(x.dtype), inter, True, arm, "w4a8_moe gemm1")
    P = sorted_ids.shape[0]
    numel = topk_ids.numel()

    lib = _abi.load()
    w2s = w2_scales.contiguous()
    w2z = w2_zeros.contiguous() if w2_zeros is not None else None
    # the reference's choice between its fused decode gemm2 + gather-reduce (rows summed unrounded)
    # and its unfused gemm2 (rows in x's dtype), kernels.py:836
    round_y2 = not (_MOE_G2FUSE and s2f != _abi.SCALE_E4M3 and s13f != _abi.SCALE_E4M3
                    and M <= _MOE_GEMM1_GEMV_MAX and block_m != 128)
    row_dt = x.dtype if round_y2 else torch.float32
    fuse2 = (_MOE_G2FUSE and arm == _abi.KERNEL_DECODE and M <= _MOE_G2C_MAX_TOKENS
             and lib.w4a8_moe_gemm2_combine_supported(inter, s2f, int(w2_zeros is not None), wfmt, _grp2, top_k) == 1)
    if fuse2:
        # one launch: requant of the gemm1 rows, gemm2, top-k weighted combine (slot order)
        out = torch.empty((M, K), dtype=x.dtype, device=x.device)
        engaged(f"w4a8_mi355x.moe_gemm2_combine({arm_name}{e2})")
        _moe_gemm2_combine(buf2, topk_ids, topk_weights, inv, M, top_k, block_m, P, t2, E, K, inter, w2s, s2f, w2z,
                           wfmt, _grp2, out, row_dt)
        return {"out": out, "buf1": buf1, "buf2": buf2, "y2": None, "topk_weights": topk_weights, "topk_ids": topk_ids,
                "sorted_ids": sorted_ids, "expert_ids": expert_ids, "ntp": ntp, "inv_pos": inv, "block_m": block_m,
                "fused_gemm2": True, "round_y2": round_y2}

    # gemm2 on the (P, inter) buffer in x's dtype, as the reference's prefill gemm2 takes it
    # (kernels.py:851-874): per-row fp8 re-quant (rows bounded by ntp on the device) into a workspace,
    # then the grouped GEMM; gemm2's (P, K) rows in the dtype the reference hands them over in
    # (above), which the combine sums in f32
    ydt = row_dt if y2_dtype is None else y2_dtype
    y2 = torch.empty((P, K), dtype=ydt, device=x.device)
    engaged(f"w4a8_mi355x.moe_gemm2({arm_name}{e2})")
    ws_bytes = int(lib.w4a8_moe_gemm_quant_workspace_bytes(P, inter))
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=x.device)
    _abi.check(
        lib.w4a8_moe_gemm_quant(_abi.ptr(buf2), _abi.dtype_code(x.dtype), inter, _abi.ptr(sorted_ids),
                                _abi.ptr(expert_ids), _abi.ptr(ntp), numel, block_m, P, _abi.ptr(t2), E, K, inter,
                                _abi.ptr(w2s), s2f, _abi.ptr(w2z), wfmt, _grp2, _abi.ptr(y2), _abi.dtype_code(ydt), K,
                                _abi.ptr(ws), ws_bytes, arm, _abi.stream_of(x)),
        "w4a8_moe gemm2")
    out = torch.empty((M, K), dtype=x.dtype, device=x.device)
    engaged("w4a8_mi355x.moe_combine")
    _abi.check(lib.w4a8_moe_combine(_abi.ptr(y2), _abi.dtype_code(ydt), K, _abi.ptr(inv), _abi.ptr(topk_weights), M,
                                    top_k, K, _abi.ptr(out), _abi.dtype_code(x.dtype), _abi.stream_of(x)),
               "w4a8_moe combine")
    return {"out": out, "buf1": buf1, "buf2": buf2, "y2": y2, "topk_weights": topk_weights, "topk_ids": topk_ids,
            "sorted_ids": sorted_ids, "expert_ids": expert_ids, "ntp": ntp, "inv_pos": inv, "block_m": block_m,
            "fused_gemm2": False, "round_y2": ydt != torch.float32}


def _w4a16_moe_forward(x, w13, w13_scales, w13_zeros, w2, w2_scales, w2_zeros, *, dt, topk_weights=None,
                       topk_ids=None, router_logits=None, top_k=0, renormalize=False, weight_is_e2m1=False,
                       block_m=None, keep_h=False, what="w4a16_moe") -> dict:
    """The grouped W4A16 MoE on the W4A8 kernels; returns the output and the intermediates.

    The activations (x in `dt`) are never rounded to fp8: each token row is split exactly into
    T = 2 (bf16) or 3 (fp16) fp8 rows (w4a16_act_split) and the route is widened to T virtual
    tokens per token (virtual token T*m + t: token m's experts, split row T*m + t), so gemm1 is the
    ordinary grouped GEMM with f32 output. w4a16_moe_silu_split sums each slot's T gate|up rows,
    applies silu * up in `dt` and splits the result back into T fp8 rows at the same padded
    positions; gemm2 runs over the same route (f32 out), and the combine weighs the T*top_k rows of
    a token with its top-k weights repeated per term."""
    M, K = x.shape
    E = w13.shape[0]
    _grp = (K // w13_scales.shape[1]) if w13_scales.dim() == 3 else -1
    assert _grp in (16, 32, 64, 128), (
        f"{what}: derived group_size={_grp} from K={K} and G={w13_scales.shape[1]}; scales must be GROUP-major "
        f"(E, K//group, N), got {tuple(w13_scales.shape)}")
    _check_moe_scale_pair(w13, w13_scales, w13_zeros, "w13")
    _check_moe_scale_pair(w2, w2_scales, w2_zeros, "w2")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"{what}: x must be bf16/fp16, got {x.dtype}")
    N1 = _n_of(w13)
    inter = N1 // 2
    if _n_of(w2) != K:
        raise AssertionError(f"{what}: w2 has {_n_of(w2)} output channels, expected hidden size {K}")
    _grp2 = inter // w2_scales.shape[1]
    if topk_ids is None:
        assert router_logits is not None and top_k > 0, (
            f"{what} needs a precomputed route (topk_ids/topk_weights) or router_logits + top_k")
        topk_weights, topk_ids = _moe_route(router_logits, top_k, renormalize, E)
    else:
        assert topk_weights is not None, "topk_weights required when topk_ids is given"
        topk_weights = topk_weights.to(torch.float32).contiguous()
        topk_ids = topk_ids.to(torch.int32).contiguous()
    top_k = topk_ids.shape[1]
    nt = 2 if dt == torch.bfloat16 else 3
    xa, xsc = w4a16_act_split(x.to(dt))
    ids_v = topk_ids.repeat_interleave(nt, dim=0).contiguous()  # (nt*M, top_k)
    numel = ids_v.numel()
    if block_m is None:
        block_m = _moe_block_m_auto(nt * M, E, top_k)
    engaged("w4a8_mi355x.moe_align")
    sorted_ids, expert_ids, ntp, inv = _moe_align(ids_v, E, block_m)
    P = sorted_ids.shape[0]

    wfmt = _abi.W_E2M1 if weight_is_e2m1 else _abi.W_INT4
    t13 = _as_tiles(w13, K, weight_is_e2m1, 3, f"{what} w13")
    t2 = _as_tiles(w2, inter, weight_is_e2m1, 3, f"{what} w2")
    s13f = _scale_fmt(w13_scales, weight_is_e2m1, f"{what} w13", w13_zeros is not None)
    s2f = _scale_fmt(w2_scales, weight_is_e2m1, f"{what} w2", w2_zeros is not None)
    if s13f == _abi.SCALE_E4M3:
        w13_scales = w13_scales.view(torch.uint8)
    if s2f == _abi.SCALE_E4M3:
        w2_scales = w2_scales.view(torch.uint8)
    arm = _abi.KERNEL_DECODE if block_m < 64 else _abi.KERNEL_PREFILL
    arm_name = "gemv" if arm == _abi.KERNEL_DECODE else "mfma"
    e2 = "+e2m1" if weight_is_e2m1 else ""
    dev = x.device

    y1 = torch.empty((P, N1), dtype=torch.float32, device=dev)
    engaged(f"w4a8_mi355x.w4a16_moe_gemm1({arm_name}{e2})")
    _moe_gemm(xa, K, xsc, 1, sorted_ids, expert_ids, ntp, numel, top_k, block_m, P, t13, E, N1, K,
              w13_scales.contiguous(), s13f, w13_zeros.contiguous() if w13_zeros is not None else None, wfmt, _grp,
              y1, _abi.F32, N1, False, arm, f"{what} gemm1")
    q2 = torch.empty((P, inter), dtype=torch.uint8, device=dev)
    s2 = torch.empty((P,), dtype=torch.float32, device=dev)
    h = torch.empty((M * top_k, inter), dtype=dt, device=dev) if keep_h else None
    lib = _abi.load()
    engaged("w4a8_mi355x.w4a16_moe_silu_split")
    _abi.check(lib.w4a16_moe_silu_split(_abi.ptr(y1), N1, _abi.ptr(inv), M, top_k, inter, _abi.dtype_code(dt),
                                        _abi.ptr(q2), inter, _abi.ptr(s2), _abi.ptr(h), inter, _abi.stream_of(x)),
               f"{what} silu_split")
    y2 = torch.empty((P, K), dtype=torch.float32, device=dev)
    engaged(f"w4a8_mi355x.w4a16_moe_gemm2({arm_name}{e2})")
    _moe_gemm(q2, inter, s2, 0, sorted_ids, expert_ids, ntp, numel, top_k, block_m, P, t2, E, K, inter,
              w2_scales.contiguous(), s2f, w2_zeros.contiguous() if w2_zeros is not None else None, wfmt, _grp2,
              y2, _abi.F32, K, False, arm, f"{what} gemm2")
    # combine over the T*top_k virtual slots of each token: slot (T*m + t, j) sits at
    # inv[m*(T*top_k) + t*top_k + j] and carries weight topk_weights[m, j]
    tw_v = topk_weights.repeat(1, nt).contiguous()
    out = torch.empty((M, K), dtype=x.dtype, device=dev)
    engaged("w4a8_mi355x.moe_combine")
    _abi.check(lib.w4a8_moe_combine(_abi.ptr(y2), _abi.F32, K, _abi.ptr(inv), _abi.ptr(tw_v), M, nt * top_k, K, _abi.ptr(out),
                                    _abi.dtype_code(x.dtype), _abi.stream_of(x)), f"{what} combine")
    return {"out": out, "h": h, "topk_weights": topk_weights, "topk_ids": topk_ids, "sorted_ids": sorted_ids,
            "expert_ids": expert_ids, "ntp": ntp, "inv_pos": inv, "block_m": block_m, "terms": nt}


def w4a16_moe(
    x: torch.Tensor,  # (M, K) activations, never quantized (cast to fp16 as the reference does)
    w13: torch.Tensor,  # (E, 2*inter, K//8) i32 op layout (gate | up), or W4 tiles
    w13_scales: torch.Tensor,  # (E, K//g, 2*inter) group-major fp16, or uint8 E8M0 (e2m1)
    w13_zeros: torch.Tensor | None,  # (E, K//g, 2*inter/8) i32 AWQ zeros | None (symmetric)
    w2: torch.Tensor,  # (E, K, inter//8) i32 op layout, or W4 tiles
    w2_scales: torch.Tensor,  # (E, inter//g, K)
    w2_zeros: torch.Tensor | None,
    hidden: int,
    inter: int,
    group_size: int,
    *,
    topk_weights: torch.Tensor | None = None,
    topk_ids: torch.Tensor | None = None,
    router_logits: torch.Tensor | None = None,
    top_k: int = 0,
    renormalize: bool = False,
    weight_is_e2m1: bool = False,
) -> torch.Tensor:
    """Grouped W4A16 MoE (python/minisgl/quant/kernels.py:899-1012): x cast to fp16 and never
    quantized, route (precomputed, or softmax + top-k from router_logits), gemm1 with silu(gate) *
    up rounded to fp16, gemm2 on those fp16 activations, top-k weighted combine in f32, cast to x's
    dtype. int4 (symmetric or with AWQ zeros) or MXFP4 (weight_is_e2m1) weights, the same tiles and
    scales as w4a8_moe. Returns (M, hidden)."""
    if x.shape[1] != hidden:
        raise AssertionError(f"w4a16_moe: hidden={hidden} does not match x's {x.shape[1]} columns")
    if _n_of(w13) != 2 * inter:
        raise AssertionError(f"w4a16_moe: inter={inter} does not match w13's {_n_of(w13)} rows (2*inter)")
    derived = hidden // w13_scales.shape[1] if w13_scales.dim() == 3 else -1
    if derived != group_size:
        raise AssertionError(f"w4a16_moe: group_size={group_size} does not match the scales' {derived}")
    return _w4a16_moe_forward(x, w13, w13_scales, w13_zeros, w2, w2_scales, w2_zeros, dt=torch.float16,
                              topk_weights=topk_weights, topk_ids=topk_ids, router_logits=router_logits, top_k=top_k,
                              renormalize=renormalize, weight_is_e2m1=weight_is_e2m1)["out"]


def w4a16_moe_decode(
    x: torch.Tensor,  # (M, K) bf16/fp16 activations, never quantized, kept in their dtype
    w13_op: torch.Tensor,  # (E, 2*inter, K//8) i32 e2m1 codes, or W4 tiles
    w13_scales: torch.Tensor,  # (E, K//16, 2*inter) e4m3 block scales, group-major
    w13_global: torch.Tensor,  # (E, 2*inter) f32 global bitcast to int32
    w2_op: torch.Tensor,  # (E, K, inter//8)
    w2_scales: torch.Tensor,  # (E, inter//16, K)
    w2_global: torch.Tensor,  # (E, K)
    hidden: int,
    *,
    topk_weights: torch.Tensor | None = None,
    topk_ids: torch.Tensor | None = None,
    router_logits: torch.Tensor | None = None,
    top_k: int = 0,
    renormalize: bool = False,
) -> torch.Tensor:
    """Grouped W4A16 MoE for NVFP4 experts (python/minisgl/quant/kernels.py:1015-1122): x in its own
    dtype and never quantized, silu(gate) * up rounded to that dtype, gemm2 on it, top-k weighted
    combine in f32, cast to x's dtype. The (E, N) globals ride the zeros slot as in w4a8_moe.
    Returns (M, hidden)."""
    for nm, t in (("w13_op", w13_op), ("w13_scales", w13_scales), ("w13_global", w13_global), ("w2_op", w2_op),
                  ("w2_scales", w2_scales), ("w2_global", w2_global)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"w4a16_moe_decode: {nm} must be a Tensor, got {type(t).__name__} ({t!r})")
    assert isinstance(hidden, int), f"hidden must be int, got {type(hidden).__name__} ({hidden!r})"
    if x.shape[1] != hidden:
        raise AssertionError(f"w4a16_moe_decode: hidden={hidden} does not match x's {x.shape[1]} columns")
    return _w4a16_moe_forward(x, w13_op, w13_scales, w13_global, w2_op, w2_scales, w2_global, dt=x.dtype,
                              topk_weights=topk_weights, topk_ids=topk_ids, router_logits=router_logits, top_k=top_k,
                              renormalize=renormalize, weight_is_e2m1=True, what="w4a16_moe_decode")["out"]
