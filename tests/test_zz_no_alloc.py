"""w4a8_linear_noalloc: the dense linear whose act-quant staging lives in the library's static
device scratch instead of a caller workspace, for callers that cannot allocate (HIP graph capture,
tight serving loops). Called through the raw C ABI and checked bit for bit against w4a8_linear with
a caller workspace, on two calls in a row per case (the second on a smaller input), and the size
refusal on the host. Named to be collected last: it must pass alone and after the other tests."""
import pytest
import torch

import synth
from conftest import pkg


def _lib():
    return pkg("_abi").load()


def _noalloc(lib, x, tiles, s, z, g, N, silu=False, kernel=0):
    abi = pkg("_abi")
    M, K = x.shape
    out = torch.empty((M, N // 2 if silu else N), dtype=x.dtype, device=x.device)
    rc = lib.w4a8_linear_noalloc(abi.ptr(x), abi.dtype_code(x.dtype), M, K, x.stride(0), abi.ptr(tiles), N,
                                 abi.ptr(s), abi.SCALE_F16, abi.ptr(z), abi.W_INT4, g, abi.ptr(out),
                                 abi.dtype_code(x.dtype), out.stride(0), int(silu), kernel, abi.stream_of(x))
    abi.check(rc, "w4a8_linear_noalloc")
    return out


def test_noalloc_refuses_oversize_on_host():
    """Sizes past the static scratch are refused before any device call, with the limit named."""
    lib = _lib()
    cap = int(lib.w4a8_linear_noalloc_max_bytes())
    assert cap == 64 << 20
    K = 4096
    M = cap // K + 1
    rc = lib.w4a8_linear_noalloc(16, 0, M, K, K, 16, 128, 16, 0, None, 0, 128, 16, 0, 128, 0, 0, None)
    assert rc != 0
    msg = lib.w4a8_last_error().decode()
    assert "static scratch" in msg and str(cap) in msg


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,g,asym", [(4096, 1024, 128, False), (2560, 768, 128, True)])
def test_noalloc_matches_workspace_entry(kernels, dev, K, N, g, asym):
    """Per case two calls in a row, the second with fewer rows: each equals w4a8_linear with a
    torch-allocated workspace bit for bit. Covers the prefill arm (act quant into the scratch), the
    decode arm on the act-quant kernel (rows > 2), the one-launch fused-quant decode call (which
    needs no scratch) and the fused SiLU arm."""
    lib = _lib()
    w, s, z = synth.int4_weight(N, K, g, seed=K + N, asym=asym, scale_floor=1e-4)
    tiles = kernels.repack_w4(w.to(dev))
    sd, zd = s.to(dev), None if z is None else z.to(dev)
    for M0, M1 in ((300, 40), (16, 5), (1, 1)):
        for M in (M0, M1):
            x = synth.activations(M, K, seed=M + K, outliers=True).to(dev)
            got = _noalloc(lib, x, tiles, sd, zd, g, N)
            ref = kernels.w4a8_linear(x, tiles, sd, zd, g)
            torch.cuda.synchronize()
            assert torch.equal(got, ref), f"M={M}: noalloc differs from w4a8_linear"
            if M <= 16:  # the fused SiLU arm is decode-only
                got_s = _noalloc(lib, x, tiles, sd, zd, g, N, silu=True)
                ref_s = kernels.w4a8_linear_silu(x, tiles, sd, zd, g)
                torch.cuda.synchronize()
                assert torch.equal(got_s, ref_s), f"M={M}: noalloc silu differs"

@pytest.mark.gpu
def test_noalloc_wide_prefill_matches_workspace_entry(kernels, dev):
    """Wide symmetric int4 prefill: with room in the static scratch the call quantizes into the
    GEMM's operand order as w4a8_linear does (1100 rows); where only the row-major codes fit (8192
    x 4096: 33.5 MB of codes, twice that with the operand-order copy) it runs the row-major GEMM.
    Both equal w4a8_linear with a torch workspace bit for bit, twice in a row."""
    lib = _lib()
    for M, K, N in ((1100, 1024, 16384), (8192, 4096, 16384), (1100, 1024, 16384)):
        w, s, _ = synth.int4_weight(N, K, 128, seed=N + K, asym=False)
        tiles, sd = kernels.repack_w4(w.to(dev)), s.to(dev)
        x = synth.activations(M, K, seed=M, outliers=True).to(dev)
        got = _noalloc(lib, x, tiles, sd, None, 128, N)
        ref = kernels.w4a8_linear(x, tiles, sd, None, 128)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"M={M} K={K}: noalloc differs from w4a8_linear"
