"""GPU parity of NVFP4 (e2m1 weights, e4m3 block-16 scales, per-output-channel f32 global) on the
dense W4A8 and W4A16 arms, through the C ABI.

NVFP4 rides the e2m1 kernels with 16-wide groups (two MFMAs per 32-element block, each on half the
block's codes) and the two-level scale of python/minisgl/quant/nvfp4.py:12-41 kept as two levels
(the accurate "split" form): the e4m3 block scale times the global, which travels in the zeros
slot as an (N,) f32 vector. Bars as for the other formats: 2e-3 relative L2 against the f64 oracle
plus the element-wise structural guard; the fused silu arm bit-identical to the unfused one.
"""
import numpy as np
import pytest
import torch

import synth
from test_gpu_dense import assert_close_to_oracle

pytestmark = pytest.mark.gpu


def _sync():
    torch.cuda.synchronize()


def _w4a8_ref(oracle, x, w, s, glob):
    xq, xs = oracle.act_quant(synth.bits16(x), 0 if x.dtype == torch.bfloat16 else 1)
    return oracle.gemm(xq, xs, w.numpy(), s.view(torch.uint8).numpy(), glob.numpy(), 16, e2m1=True, nvfp4=True)


def _w4a16_ref(oracle, x, w, s, glob):
    return oracle.w4a16_gemm(synth.bits16(x), 0 if x.dtype == torch.bfloat16 else 1, w.numpy(),
                             s.view(torch.uint8).numpy(), glob.numpy(), 16, e2m1=True, nvfp4=True)


@pytest.mark.parametrize("K,N", [(1024, 512), (4096, 1536)])
def test_nvfp4_w4a8_matches_oracle(kernels, oracle, dev, K, N):
    w, s, glob = synth.nvfp4_weight(N, K, seed=K + N)
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=True)
    sd, gd = s.to(dev), glob.to(dev)
    for M in (1, 3, 16, 17, 64, 200):  # decode GEMV and tiled arms
        x = synth.activations(M, K, seed=M, outliers=True)
        out = kernels.w4a8_linear(x.to(dev), tiles, sd, gd, 16, weight_is_e2m1=True)
        _sync()
        assert_close_to_oracle(out, _w4a8_ref(oracle, x, w, s, glob), f"nvfp4 w4a8 K={K} N={N} M={M}")


@pytest.mark.parametrize("K,N", [(2048, 1536), (8192, 512)])
def test_nvfp4_prefill_fp16_mfma(kernels, oracle, dev, K, N):
    """The prefill arm runs NVFP4 on the fp16 MFMA (e2m1 * e4m3 block scale and the e4m3
    activation codes are exact in fp16): against the oracle at 2e-3 with the structural guard on
    every row of M = 640 (a partial 256-row tile; 64-row tiles for the small grid of N = 512), and
    row-split invariant bit for bit (rows 200..263 alone, a different tile shape, equal the same
    rows of the full call)."""
    w, s, glob = synth.nvfp4_weight(N, K, seed=K // 64 + N)
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=True)
    sd, gd = s.to(dev), glob.to(dev)
    x = synth.activations(640, K, seed=K, outliers=True)
    out = kernels.w4a8_linear(x.to(dev), tiles, sd, gd, 16, weight_is_e2m1=True)
    part = kernels.w4a8_linear(x[200:264].to(dev), tiles, sd, gd, 16, weight_is_e2m1=True)
    _sync()
    assert torch.equal(part, out[200:264])
    assert_close_to_oracle(out, _w4a8_ref(oracle, x, w, s, glob), f"nvfp4 prefill K={K} N={N} M=640")


def test_nvfp4_scale_dtype_forms_agree(kernels, dev):
    """float8_e4m3fn scales, their uint8 bytes (+ populated zeros slot) and the global as f32 or as its
    int32 bit pattern are the same call (python/minisgl/quant/kernels.py:518-559)."""
    K, N = 512, 256
    w, s, glob = synth.nvfp4_weight(N, K, seed=3)
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=True)
    x = synth.activations(5, K, seed=3).to(dev)
    a = kernels.w4a8_linear(x, tiles, s.to(dev), glob.to(dev), 16, weight_is_e2m1=True)
    b = kernels.w4a8_linear(x, tiles, s.view(torch.uint8).to(dev), glob.view(torch.int32).to(dev), 16,
                            weight_is_e2m1=True)
    _sync()
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_nvfp4_w4a16_matches_oracle(kernels, oracle, dev, dtype):
    K, N = 1024, 512
    w, s, glob = synth.nvfp4_weight(N, K, seed=11)
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=True)
    sd, gd = s.to(dev), glob.to(dev)
    for M in (1, 8, 17, 64, 200):
        x = (synth.activations(M, K, seed=M + 1, dtype=torch.float32) * 0.5).to(dtype)
        out = kernels.w4a16_linear(x.to(dev), tiles, sd, gd, 16, N, weight_is_e2m1=True)
        _sync()
        assert out.dtype == dtype
        assert_close_to_oracle(out, _w4a16_ref(oracle, x, w, s, glob), f"nvfp4 w4a16 {dtype} M={M}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_nvfp4_fused_silu_bit_exact(kernels, dev, dtype):
    inter, K = 512, 768
    N = 2 * inter
    w, s, glob = synth.nvfp4_weight(N, K, seed=13)
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=True)
    sd, gd = s.to(dev), glob.to(dev)
    for M in (1, 4):
        x = (synth.activations(M, K, seed=M, dtype=torch.float32) * 0.3).to(dtype).to(dev)
        full = kernels.w4a8_linear(x, tiles, sd, gd, 16, kernel="decode_gemv", weight_is_e2m1=True)
        gh, uh = full[:, :inter], full[:, inter:]
        ref = (gh.float() / (1.0 + torch.exp(-gh.float()))).to(dtype) * uh
        fused = kernels.w4a8_linear_silu(x, tiles, sd, gd, 16, weight_is_e2m1=True)
        _sync()
        assert torch.equal(fused, ref)


def test_nvfp4_w4a16_no_further_from_exact_than_w4a8(kernels, oracle, dev):
    """The reference's tests/w4a16_e2m1_parity_test.py NVFP4 g=16 case, directionally."""
    K, N = 2048, 256
    w, s, glob = synth.nvfp4_weight(N, K, seed=17)
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=True)
    sd, gd = s.to(dev), glob.to(dev)
    for M in (1, 17, 200):
        x = synth.activations(M, K, seed=M, outliers=True)
        exact = _w4a16_ref(oracle, x, w, s, glob)
        a16 = kernels.w4a16_linear(x.to(dev), tiles, sd, gd, 16, N, weight_is_e2m1=True).float().cpu().numpy()
        a8 = kernels.w4a8_linear(x.to(dev), tiles, sd, gd, 16, weight_is_e2m1=True).float().cpu().numpy()
        assert np.linalg.norm(a16 - exact) <= np.linalg.norm(a8 - exact)


@pytest.mark.parametrize("T,bm", [(8, 16), (64, 64), (512, 128)])
def test_nvfp4_moe(kernels, oracle, dev, T, bm):
    """NVFP4 experts (e2m1 + e4m3 block-16 + (E, N) global in the zeros slot) through the grouped
    kernels (python/minisgl/quant/kernels.py:484-559), decode and tiled arms; stage by stage and end
    to end within what the stages and the contract's requant amplification account for (as in
    test_gpu_moe), on up to 32 tokens."""
    from test_gpu_moe import _assert_end_to_end, _stagewise, _subset

    top_k, e, h, i = 4, 32, 1024, 512
    w13, s13, g13 = synth.nvfp4_weight(2 * i, h, seed=451, E=e)
    w2, s2, g2 = synth.nvfp4_weight(h, i, seed=452, E=e)
    x = synth.activations(T, h, seed=453 + T)
    lg = synth.router_logits(T, e, seed=454 + T)
    res = kernels._moe_forward(x.to(dev), w13.to(dev), s13.to(dev), g13.view(torch.int32).to(dev), w2.to(dev),
                               s2.to(dev), g2.view(torch.int32).to(dev), lg.to(dev), top_k, True, block_m=bm,
                               weight_is_e2m1=True)
    _sync()
    out = res["out"]
    subl = _subset(T)
    rel1, rel2, y2ref = _stagewise(kernels, oracle, res, x, w13, s13.view(torch.uint8), g13, w2, s2.view(torch.uint8),
                                     g2, subl, e2m1=True, nvfp4=True)
    assert rel1 <= 2e-3 and rel2 <= 2e-3, f"nvfp4 moe T={T} bm={bm}: stages {rel1:.3e} {rel2:.3e}"
    sub = torch.tensor(subl)
    tw, ids = oracle.moe_route(lg[sub].float().numpy(), top_k, True)
    sorted_ids, expert_ids, ntp, _ = oracle.moe_align(ids, e, 16)
    ref = oracle.moe_forward(synth.bits16(x[sub]), 0, tw, sorted_ids, expert_ids, ntp, 16, top_k, w13.numpy(),
                             s13.view(torch.uint8).numpy(), g13.numpy(), w2.numpy(), s2.view(torch.uint8).numpy(),
                             g2.numpy(), e2m1=True, nvfp4=True, round_y2=res["round_y2"])
    _assert_end_to_end(out[sub.to(dev)], ref, y2ref, rel2, f"nvfp4 moe T={T} bm={bm}")
