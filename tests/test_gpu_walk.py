"""GPU: the strip-walking decode GEMV, which quantizes a decode call's bf16/fp16 rows itself (one
launch for up to 16 rows), against the two-launch path (act quant, then the GEMV on the fp8 pair).

The two paths must agree bit for bit: the walker keeps the one-row K split, the per-tile MFMA/FMA
steps and the wave-order reduction of the GEMV, and its row phase is the act-quant kernel's
arithmetic. The two-launch path is itself held to the oracle (test_gpu_dense.py), so this pins the
walker to the oracle's contract as well; a few calls are also checked against the oracle directly.
"""
import pytest
import torch

import synth
from conftest import pkg
from test_gpu_dense import _oracle_dense, assert_close_to_oracle

pytestmark = pytest.mark.gpu

# (K, N, format): the configs[1] shapes, configs[0], MXFP4 at configs[5]'s down shape, a 5-wave and
# a 6-wave K split (threads per row not a power of two), a one-tile K, an N that is not a multiple
# of 32, a two-strip weight, and NVFP4 (which walks above 4 rows)
CASES = [(4096, 6144, "sym"), (4096, 4096, "sym"), (4096, 28672, "sym"), (14336, 4096, "sym"),
         (2560, 9728, "asym"), (28672, 8192, "e2m1"), (1536, 768, "e2m1"), (2048, 9600, "sym"),
         (128, 64, "sym"), (384, 4112, "asym"), (1024, 32, "asym"), (8192, 28672, "nvfp4"), (2048, 768, "nvfp4")]
MS = (1, 2, 3, 4, 5, 7, 8, 9, 13, 16)


def _weights(K, N, fmt, dev, seed):
    e2 = fmt in ("e2m1", "nvfp4")
    if fmt == "nvfp4":
        w, s, gl = synth.nvfp4_weight(N, K, seed=seed)
        z, g = gl, 16
    elif e2:
        w, s = synth.mxfp4_weight(N, K, seed=seed)
        z, g = None, 32
    else:
        g = 128
        w, s, z = synth.int4_weight(N, K, g, seed=seed, asym=fmt == "asym", scale_floor=1e-4)
    kernels = pkg("quant.kernels")
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=e2)
    return w, s, z, g, e2, tiles, s.to(dev), None if z is None else z.to(dev)


def _launches(lib, M, K, N, fmt, dtype, silu=False):
    e2 = fmt in ("e2m1", "nvfp4")
    sfmt = 2 if fmt == "nvfp4" else 1 if e2 else 0
    return lib.w4a8_linear_launch_count(M, N, K, 0 if dtype == torch.bfloat16 else 1, sfmt,
                                        int(fmt in ("asym", "nvfp4")), int(e2), 16 if fmt == "nvfp4" else 32 if e2 else 128,
                                        int(silu), 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K,N,fmt", CASES)
def test_walk_matches_two_launch_path(kernels, dev, K, N, fmt, dtype):
    lib = pkg("_abi").load()
    _, _, _, g, e2, tiles, sd, zd = _weights(K, N, fmt, dev, seed=N + 3)
    x = synth.activations(16, K, seed=K + N, outliers=True, dtype=dtype).to(dev)
    single = 0
    for m in MS:
        xm = x[:m].contiguous()
        q, sc = kernels.act_quant(xm)
        a = kernels.w4a8_linear(xm, tiles, sd, zd, g, weight_is_e2m1=e2)
        b = kernels.w4a8_linear(xm, tiles, sd, zd, g, weight_is_e2m1=e2, x_fp8=q, act_scales=sc)
        torch.cuda.synchronize()
        single += _launches(lib, m, K, N, fmt, dtype) == 1
        assert torch.equal(a, b), f"K={K} N={N} {fmt} {dtype} M={m}: max|d| {(a.float() - b.float()).abs().max().item():.3e}"
    assert single > 0, "no call took the one-launch path"


@pytest.mark.parametrize("K,N,fmt", [(4096, 28672, "sym"), (2560, 9728, "asym"), (1536, 768, "e2m1"),
                                     (14336, 4096, "sym")])
def test_walk_silu_matches_unfused(kernels, dev, K, N, fmt):
    """The fused silu arm of the walker against the plain arm on the fp8 pair plus the
    round-silu-round-multiply replica (tools/w4a8_gemm_silu_parity.py:52-54), bit for bit."""
    _, _, _, g, e2, tiles, sd, zd = _weights(K, N, fmt, dev, seed=N + 5)
    inter = N // 2
    for dtype in (torch.bfloat16, torch.float16):
        x = (synth.activations(16, K, seed=K + 1, dtype=torch.float32) * 0.3).to(dtype).to(dev)
        for m in (1, 2, 4, 8, 16):
            xm = x[:m].contiguous()
            q, sc = kernels.act_quant(xm)
            y = kernels.w4a8_linear(xm, tiles, sd, zd, g, kernel="decode_gemv", weight_is_e2m1=e2, x_fp8=q,
                                    act_scales=sc)
            gh, uh = y[:, :inter], y[:, inter:]
            ref = (gh.float() / (1.0 + torch.exp(-gh.float()))).to(dtype) * uh
            fused = kernels.w4a8_linear_silu(xm, tiles, sd, zd, g, weight_is_e2m1=e2)
            torch.cuda.synchronize()
            assert torch.equal(fused, ref), f"K={K} N={N} {fmt} {dtype} M={m}"


def test_walk_special_rows(kernels, dev):
    """Rows of zeros, rows whose maximum is exactly 448, rows of bf16 subnormals and rows holding +-inf
    or NaN: the walker's packed-magnitude maximum (and its f32 fallback for NaN) gives the act-quant
    kernel's codes, so the outputs equal the two-launch path's bit for bit (NaN payloads included)."""
    K, N = 4096, 4096
    _, _, _, g, e2, tiles, sd, zd = _weights(K, N, "sym", dev, seed=11)
    x = synth.activations(8, K, seed=3).float()
    x[0] = 0.0
    x[1, 17] = 448.0
    x[1].clamp_(-448.0, 448.0)
    x[2] = torch.full((K,), 2.0 ** -130) * torch.sign(torch.randn(K))
    x[3, 100] = float("inf")
    x[4, 5] = float("-inf")
    x[5, 7] = float("nan")
    x[6, :] = float("nan")
    x = x.to(torch.bfloat16).to(dev)
    q, sc = kernels.act_quant(x)
    a = kernels.w4a8_linear(x, tiles, sd, zd, g)
    b = kernels.w4a8_linear(x, tiles, sd, zd, g, x_fp8=q, act_scales=sc)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_walk_against_oracle(kernels, oracle, dev):
    """Walked calls at configs[1]'s gate_up and down shapes against the oracle directly."""
    for K, N in [(4096, 28672), (14336, 4096)]:
        w, s, _, g, _, tiles, sd, _ = _weights(K, N, "sym", dev, seed=K)
        x = synth.activations(4, K, seed=N, outliers=True)
        ref = _oracle_dense(oracle, x, w, s, None, g)
        out = kernels.w4a8_linear(x.to(dev), tiles, sd, None, g)
        torch.cuda.synchronize()
        assert pkg("_abi").load().w4a8_linear_launch_count(4, N, K, 0, 0, 0, 0, 128, 0, 0) == 1
        assert_close_to_oracle(out, ref, f"walk K={K} N={N} M=4")
