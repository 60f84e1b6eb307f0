"""GPU: the decode GEMV's fused activation quant (bf16/fp16 rows quantized per token in the
kernel's prologue) against the two-launch path (act-quant kernel, then the GEMM on the fp8 pair).

Bar: bit-identical outputs. The fused prologue runs the act-quant kernel's arithmetic (amax,
s = max(amax/448, 1e-8), IEEE 1/s, RNE e4m3) and the GEMV's K split does not depend on where A
comes from, so any difference is a bug. The two-launch path is itself pinned to the oracle by
test_gpu_dense.py.
"""
import pytest
import torch

import synth
from conftest import pkg

pytestmark = pytest.mark.gpu


def _weights(kernels, dev, fmt, N, K, seed):
    if fmt == "e2m1":
        w, s = synth.mxfp4_weight(N, K, seed=seed)
        return kernels.repack_w4(w.to(dev), weight_is_e2m1=True), s.to(dev), None, 32, True
    g = 128
    w, s, z = synth.int4_weight(N, K, g, seed=seed, asym=fmt == "asym")
    return kernels.repack_w4(w.to(dev)), s.to(dev), (None if z is None else z.to(dev)), g, False


CASES = [(M, K) for M in (1, 2, 3, 4, 5, 8, 16) for K in (256, 1024, 4096)] + \
        [(1, 14336), (2, 14336), (1, 2880), (3, 2880), (1, 8192), (4, 8192)]


@pytest.mark.parametrize("fmt", ["sym", "asym", "e2m1"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_quant_matches_two_launch(kernels, dev, fmt, dtype):
    N = 256
    for (M, K) in CASES:
        if fmt != "e2m1" and K % 128:
            continue
        tiles, s, z, g, e2 = _weights(kernels, dev, fmt, N, K, seed=M + K)
        x = synth.activations(M, K, seed=3 * M + K, dtype=torch.float32).to(dtype).to(dev)
        x[0, :] = 0  # an all-zero row takes the 1e-8 scale floor
        q, sc = kernels.act_quant(x)
        fused = kernels.w4a8_linear(x, tiles, s, z, g, kernel="decode_gemv", weight_is_e2m1=e2)
        pair = kernels.w4a8_linear(x, tiles, s, z, g, kernel="decode_gemv", weight_is_e2m1=e2, x_fp8=q,
                                   act_scales=sc)
        torch.cuda.synchronize()
        assert torch.equal(fused, pair), f"{fmt} {dtype} M={M} K={K}: max " \
                                         f"{(fused.float() - pair.float()).abs().max().item():.3e}"


def _launches(lib, M, N, K, e2):
    return lib.w4a8_linear_launch_count(M, N, K, 0, 1 if e2 else 0, 0, int(e2), 32 if e2 else 128, 0, 1)


@pytest.mark.parametrize("M,K", [(1, 4096), (2, 4096), (4, 4096), (8, 4096), (1, 14336), (4, 14336), (1, 2880)])
def test_fused_quant_is_one_launch(kernels, dev, M, K):
    """Decode calls whose rows the GEMV quantizes itself (the one-row fused prologue, or the
    strip-walking GEMV for up to 16 rows) run without a workspace (no act-quant launch): the ABI
    refuses a null workspace whenever it would need one, and the planner query agrees."""
    abi = pkg("_abi")
    lib = abi.load()
    N = 128
    fmt = "e2m1" if K % 128 else "sym"
    tiles, s, z, g, e2 = _weights(kernels, dev, fmt, N, K, seed=K)
    assert _launches(lib, M, N, K, e2) == 1
    x = synth.activations(M, K, seed=M).to(dev)
    out = torch.empty((M, N), dtype=x.dtype, device=dev)
    rc = lib.w4a8_linear(abi.ptr(x), abi.BF16, M, K, K, abi.ptr(tiles), N, abi.ptr(s),
                         abi.SCALE_E8M0 if e2 else abi.SCALE_F16, None, abi.W_E2M1 if e2 else abi.W_INT4, g,
                         abi.ptr(out), abi.BF16, N, 0, None, 0, abi.KERNEL_DECODE, abi.stream_of(x))
    assert rc == 0, lib.w4a8_last_error().decode()
    ref = kernels.w4a8_linear(x, tiles, s, z, g, kernel="decode_gemv", weight_is_e2m1=e2,
                              x_fp8=kernels.act_quant(x)[0], act_scales=kernels.act_quant(x)[1])
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("M,K", [(16, 4096), (8, 14336)])
def test_unfused_needs_workspace(kernels, dev, M, K):
    """Calls whose row phase would cost the GEMV more than an act-quant launch (16 rows of 4096 on a
    narrow weight, 8 rows of 14336) take the act-quant kernel first: without a workspace the call
    fails loudly."""
    abi = pkg("_abi")
    lib = abi.load()
    N = 128
    tiles, s, z, g, e2 = _weights(kernels, dev, "sym", N, K, seed=5)
    assert _launches(lib, M, N, K, e2) == 2
    x = synth.activations(M, K, seed=1).to(dev)
    out = torch.empty((M, N), dtype=x.dtype, device=dev)
    rc = lib.w4a8_linear(abi.ptr(x), abi.BF16, M, K, K, abi.ptr(tiles), N, abi.ptr(s), abi.SCALE_F16, None,
                         abi.W_INT4, g, abi.ptr(out), abi.BF16, N, 0, None, 0, abi.KERNEL_DECODE, abi.stream_of(x))
    assert rc == 1  # W4A8_ERR_INVALID
    assert b"workspace" in lib.w4a8_last_error()
