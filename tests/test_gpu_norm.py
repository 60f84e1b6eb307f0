"""GPU: the RMSNorm producer (w4a8_rms_norm) and the fp8 pair it hands to the W4A8 linears.

Bars:
- out and the updated residual equal the oracle bit for bit (the oracle restates the kernel's
  documented f32 summation order; the external kernel's order is unpinned);
- the fused pair equals act_quant(out) bit for bit, and out is the same with or without the pair;
- a w4a8 linear fed the pair gives exactly what it gives when it quantizes out itself
  (tools/w4a8_producer_actquant.py:113-136), on the decode and the prefill arms.
"""
import numpy as np
import pytest
import torch

import synth
from conftest import pkg

pytestmark = pytest.mark.gpu


def _norm():
    return pkg("layers.norm")


def _bits(t):
    return synth.bits16(t.cpu())


SHAPES = [(1, 2048), (7, 4096), (33, 5120), (129, 2816), (3, 14336), (2, 8), (5, 32768)]


@pytest.mark.parametrize("dtype,code", [(torch.bfloat16, 0), (torch.float16, 1)])
@pytest.mark.parametrize("M,K", SHAPES)
def test_rms_norm_matches_oracle(oracle, dev, dtype, code, M, K):
    N = _norm()
    g = torch.Generator().manual_seed(M * 7 + K)
    x = (torch.randn(M, K, generator=g) * 0.7).to(dtype)
    x[0, :] = 0
    r = (torch.randn(M, K, generator=g) * 0.7).to(dtype)
    w = (torch.randn(K, generator=g) * 0.1 + 1.0).to(dtype)
    xd, wd = x.to(dev), w.to(dev)
    for weight, plus_one in ((w, False), (w - 1.0, True), (None, False)):
        wt = None if weight is None else weight.to(dtype)
        out = N._rms_norm(xd, None if wt is None else wt.to(dev), 1e-6, plus_one)
        ro, _ = oracle.rms_norm(_bits(x), None if wt is None else _bits(wt), 1e-6, code, plus_one)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out), ro), f"norm M={M} K={K} plus_one={plus_one} weight={weight is not None}"
    # fused residual add, with the quant epilogue
    rd = r.to(dev)
    out, q, s = N._rms_norm_add_quant(xd, rd, wd, 1e-5)
    ro, rr = oracle.rms_norm(_bits(x), _bits(w), 1e-5, code, False, residual_bits=_bits(r))
    q2, s2 = pkg("quant.kernels").act_quant(out)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(rd), rr), "residual <- x + residual"
    assert np.array_equal(_bits(out), ro), "norm over the sum"
    assert torch.equal(q, q2) and torch.equal(s, s2), "fused pair == act_quant(out)"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quant_forms_keep_out_identical(dev, dtype):
    N = _norm()
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(17, 4096, generator=g) * 0.7).to(dtype).to(dev)
    w = (torch.randn(4096, generator=g) * 0.1 + 1.0).to(dtype).to(dev)
    a = N._rms_norm(x, w, 1e-6)
    b, q, s = N._rms_norm_quant(x, w, 1e-6)
    r1 = (torch.randn(17, 4096, generator=g) * 0.7).to(dtype).to(dev)
    r2 = r1.clone()
    fused = N.RMSNormFused(4096, 1e-6)
    fused.weight = w
    o1, res1 = fused.forward(x, r1)
    o2, res2, q2, s2 = fused.forward_quant(x, r2)
    plain = N.RMSNorm(4096, 1e-6)
    plain.weight = w
    xi = x.clone()
    plain.forward_inplace(xi)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(o1, o2) and torch.equal(res1, res2) and torch.equal(xi, a)
    assert res2.data_ptr() == r2.data_ptr(), "the residual stays the same storage"


@pytest.mark.parametrize("M", [1, 2, 16, 17, 33, 129, 512])
@pytest.mark.parametrize("fmt", ["sym", "asym", "e2m1"])
def test_linear_on_the_producer_pair_is_bit_identical(kernels, dev, M, fmt):
    """The gate of tools/w4a8_producer_actquant.py:113-136: the pair the producer emitted drives the
    linear, through its auto-dispatch, to exactly the answer it gives when it quantizes itself."""
    N = _norm()
    K, Nout = 2048, 1024
    g = torch.Generator().manual_seed(M)
    x = (torch.randn(M, K, generator=g) * 0.7).to(torch.bfloat16).to(dev)
    r = (torch.randn(M, K, generator=g) * 0.7).to(torch.bfloat16).to(dev)
    w = (torch.randn(K, generator=g) * 0.1 + 1.0).to(torch.bfloat16).to(dev)
    if fmt == "e2m1":
        wq, ws = synth.mxfp4_weight(Nout, K, seed=M)
        tiles, sc, z, gs, e2 = kernels.repack_w4(wq.to(dev), weight_is_e2m1=True), ws.to(dev), None, 32, True
    else:
        wq, ws, wz = synth.int4_weight(Nout, K, 128, seed=M, asym=fmt == "asym")
        tiles, sc, gs, e2 = kernels.repack_w4(wq.to(dev)), ws.to(dev), 128, False
        z = None if wz is None else wz.to(dev)
    out, q, s = N._rms_norm_add_quant(x, r, w, 1e-6)
    base = kernels.w4a8_linear(out, tiles, sc, z, gs, weight_is_e2m1=e2)
    fused = kernels.w4a8_linear(out, tiles, sc, z, gs, weight_is_e2m1=e2, x_fp8=q, act_scales=s)
    torch.cuda.synchronize()
    assert torch.equal(base, fused), f"M={M} {fmt}: max {(base.float() - fused.float()).abs().max().item():.3e}"


def test_refusals_are_loud(dev):
    abi = pkg("_abi")
    lib = abi.load()
    x = torch.zeros(4, 64, dtype=torch.bfloat16, device=dev)
    o = torch.empty_like(x)
    q = torch.empty(4, 64, dtype=torch.uint8, device=dev)
    st = abi.stream_of(x)
    rc = lib.w4a8_rms_norm(abi.ptr(x), abi.BF16, 4, 64, 64, None, 64, None, 0, 1e-6, abi.ptr(o), 64, abi.ptr(q), 64,
                           None, st)
    assert rc == 1 and b"TOGETHER" in lib.w4a8_last_error()
    rc = lib.w4a8_rms_norm(abi.ptr(x), abi.BF16, 4, 64, 64, abi.ptr(x), 64, None, 0, 1e-6, abi.ptr(o), 64, None, 64,
                           None, st)
    assert rc == 1 and b"residual" in lib.w4a8_last_error()
    big = torch.zeros(1, 32776, dtype=torch.bfloat16, device=dev)
    rc = lib.w4a8_rms_norm(abi.ptr(big), abi.BF16, 1, 32776, 32776, None, 32776, None, 0, 1e-6, abi.ptr(big), 32776,
                           None, 32776, None, st)
    assert rc == 2 and b"32768" in lib.w4a8_last_error()
    N = _norm()
    assert N._rms_norm_quant(torch.zeros(2, 64, device=dev), None, 1e-6) is None  # f32: not the native kernel
    with pytest.raises(TypeError):
        N._rms_norm(torch.zeros(2, 64, device=dev), None, 1e-6)
