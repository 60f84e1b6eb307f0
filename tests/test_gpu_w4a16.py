"""GPU parity of the W4A16 arm (unquantized activations on the W4A8 weights), through the C ABI.

Bars: the activation split bit-exact against the CPU oracle; outputs within 2e-3 relative L2 of
the oracle's f64 x @ dequant(W)^T (with the element-wise structural guard of the dense tests); the
fused silu arm bit-identical to w4a16_linear followed by the round-silu-round-mul replica. The
directional checks of the reference's tests/w4a16_e2m1_parity_test.py:101-131 hold too: W4A16 is
no further from the unquantized product than W4A8, and keeps the activation dtype.
"""
import numpy as np
import pytest
import torch

import synth
from conftest import pkg
from test_gpu_dense import assert_close_to_oracle

pytestmark = pytest.mark.gpu


def _sync():
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype,code", [(torch.bfloat16, 0), (torch.float16, 1)])
@pytest.mark.parametrize("M,K", [(1, 4096), (3, 14336), (16, 2560), (70, 136), (257, 1024)])
def test_act_split_bit_exact(kernels, oracle, dev, dtype, code, M, K):
    x = synth.activations(M, K, seed=M + K, outliers=True, dtype=torch.float32).to(dtype)
    x[0, :8] = 0.0
    q, s = kernels.w4a16_act_split(x.to(dev))
    _sync()
    rq, rs = oracle.act_split(synth.bits16(x), code)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy(), rs)


def _case(fmt, N, K, seed):
    if fmt == "mxfp4":
        w, s = synth.mxfp4_weight(N, K, seed=seed)
        return w, s, None, 32, True
    if fmt == "e2m1_f16":
        w, s8 = synth.mxfp4_weight(N, K, seed=seed)
        return w, torch.pow(2.0, s8.float() - 127).to(torch.float16), None, 32, True
    g = 32 if fmt.endswith("g32") else 128
    w, s, z = synth.int4_weight(N, K, g, seed=seed, asym=fmt.startswith("asym"), scale_floor=1e-4)
    return w, s, z, g, False


def _oracle_ref(oracle, x, w, s, z, g, e2m1):
    return oracle.w4a16_gemm(synth.bits16(x), 0 if x.dtype == torch.bfloat16 else 1, w.numpy(), s.numpy(),
                             None if z is None else z.numpy(), g, e2m1)


@pytest.mark.parametrize("fmt", ["sym", "asym", "sym_g32", "mxfp4", "e2m1_f16"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_w4a16_linear_matches_oracle(kernels, oracle, dev, fmt, dtype):
    K, N = 1024, 512
    w, s, z, g, e2 = _case(fmt, N, K, seed=len(fmt))
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=e2)
    sd, zd = s.to(dev), None if z is None else z.to(dev)
    # M straddles the decode / tiled split (16 tokens)
    for M in (1, 3, 8, 16, 17, 64, 200):
        x = (synth.activations(M, K, seed=M + 5, outliers=True, dtype=torch.float32) * 0.5).to(dtype)
        out = kernels.w4a16_linear(x.to(dev), tiles, sd, zd, g, N, weight_is_e2m1=e2)
        _sync()
        assert out.dtype == dtype and tuple(out.shape) == (M, N)
        assert_close_to_oracle(out, _oracle_ref(oracle, x, w, s, z, g, e2), f"w4a16 {fmt} {dtype} M={M}")


@pytest.mark.parametrize("K,N", [(4096, 6144), (14336, 4096)])
def test_w4a16_llama_shapes(kernels, oracle, dev, K, N):
    w, s, _ = synth.int4_weight(N, K, 128, seed=K, asym=False)
    tiles, sd = kernels.repack_w4(w.to(dev)), s.to(dev)
    for M in (1, 16, 300):
        x = synth.activations(M, K, seed=M, outliers=True)
        out = kernels.w4a16_linear(x.to(dev), tiles, sd, None, 128, N)
        _sync()
        assert_close_to_oracle(out, _oracle_ref(oracle, x, w, s, None, 128, False), f"w4a16 K={K} N={N} M={M}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fmt", ["sym", "asym", "mxfp4"])
def test_w4a16_silu_bit_exact(kernels, dev, dtype, fmt):
    """Fused gate_up arm == w4a16_linear + round-silu-round-mul, bit for bit (python/minisgl/quant/
    kernels.py:1772-1776)."""
    inter, K = 512, 768
    N = 2 * inter
    w, s, z, g, e2 = _case(fmt, N, K, seed=9)
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=e2)
    sd, zd = s.to(dev), None if z is None else z.to(dev)
    for M in (1, 5, 40):
        x = (synth.activations(M, K, seed=M, dtype=torch.float32) * 0.3).to(dtype).to(dev)
        full = kernels.w4a16_linear(x, tiles, sd, zd, g, N, weight_is_e2m1=e2)
        gh, uh = full[:, :inter], full[:, inter:]
        ref = (gh.float() / (1.0 + torch.exp(-gh.float()))).to(dtype) * uh
        fused = kernels.w4a16_linear_silu(x, tiles, sd, zd, g, weight_is_e2m1=e2)
        _sync()
        assert fused.dtype == dtype and tuple(fused.shape) == (M, inter)
        assert torch.equal(fused, ref), f"{fmt} {dtype} M={M}: max {(fused.float() - ref.float()).abs().max().item():.3e}"


def _split_rows_f32(q, sc, tiles, s, z, g, N, K, e2):
    """The fp8 GEMM of the split rows with f32 output, through the C ABI's prefill arm."""
    abi = pkg("_abi")
    lib = abi.load()
    y = torch.empty((q.shape[0], N), dtype=torch.float32, device=q.device)
    sfmt = abi.SCALE_F16 if s.dtype == torch.float16 else abi.SCALE_E8M0
    abi.check(lib.w4a8_gemm(abi.ptr(q), K, abi.ptr(sc), q.shape[0], abi.ptr(tiles), N, K, abi.ptr(s), sfmt,
                            abi.ptr(z), abi.W_E2M1 if e2 else abi.W_INT4, g, abi.ptr(y), abi.F32, N, 0, None, 0,
                            abi.KERNEL_PREFILL, abi.stream_of(q)), "w4a8_gemm")
    return y


@pytest.mark.parametrize("fmt", ["sym", "asym", "mxfp4"])
def test_w4a16_bf16_term_sum_in_epilogue(kernels, dev, fmt):
    """bf16 prefill: the GEMM's epilogue adds each row's two fp8 terms and rounds once. Bit-identical
    to the arm composed from its pieces: w4a16_act_split, the fp8 GEMM writing the terms' f32 rows,
    and (0 + y[2m]) + y[2m+1] in f32 rounded to bf16 (the sum the decode arm's kernel takes)."""
    K, N = 1024, 512
    w, s, z, g, e2 = _case(fmt, N, K, seed=31)
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=e2)
    sd, zd = s.to(dev), None if z is None else z.to(dev)
    for M in (17, 64, 300):
        x = (synth.activations(M, K, seed=M + 3, outliers=True, dtype=torch.float32) * 0.5).to(torch.bfloat16).to(dev)
        x[1, :16] = 0.0
        out = kernels.w4a16_linear(x, tiles, sd, zd, g, N, weight_is_e2m1=e2)
        q, sc = kernels.w4a16_act_split(x)
        y = _split_rows_f32(q, sc, tiles, sd, zd, g, N, K, e2)
        ref = ((0.0 + y[0::2]) + y[1::2]).to(torch.bfloat16)
        _sync()
        assert torch.equal(out, ref), f"{fmt} M={M}: max {(out.float() - ref.float()).abs().max().item():.3e}"


@pytest.mark.parametrize("fmt", ["sym", "mxfp4"])
def test_w4a16_bf16_term_sum_wide_weights(kernels, dev, fmt):
    """The same on a wide symmetric int4 or MXFP4 weight at 600 tokens (1200 term rows): there the
    terms' codes are also rewritten in the GEMM's operand order (with the row-sum seeds for int4)
    before the GEMM, and the fused silu arm runs on the same path."""
    K, N = 1024, 16384
    w, s, _, g, e2 = _case(fmt, N, K, seed=33)
    tiles, sd = kernels.repack_w4(w.to(dev), weight_is_e2m1=e2), s.to(dev)
    M = 600
    x = (synth.activations(M, K, seed=7, outliers=True, dtype=torch.float32) * 0.5).to(torch.bfloat16).to(dev)
    out = kernels.w4a16_linear(x, tiles, sd, None, g, N, weight_is_e2m1=e2)
    q, sc = kernels.w4a16_act_split(x)
    y = _split_rows_f32(q, sc, tiles, sd, None, g, N, K, e2)
    ref = ((0.0 + y[0::2]) + y[1::2]).to(torch.bfloat16)
    inter = N // 2
    gh, uh = ref[:, :inter], ref[:, inter:]
    ref_s = (gh.float() / (1.0 + torch.exp(-gh.float()))).to(torch.bfloat16) * uh
    fused = kernels.w4a16_linear_silu(x, tiles, sd, None, g, weight_is_e2m1=e2)
    _sync()
    assert torch.equal(out, ref), f"max {(out.float() - ref.float()).abs().max().item():.3e}"
    assert torch.equal(fused, ref_s), f"silu max {(fused.float() - ref_s.float()).abs().max().item():.3e}"


@pytest.mark.parametrize("fmt", ["sym", "mxfp4"])
def test_w4a16_no_further_from_exact_than_w4a8(kernels, oracle, dev, fmt):
    """tests/w4a16_e2m1_parity_test.py:119-129 of the reference, directionally: against the
    unquantized product of the same 4-bit weights, W4A16 is no further off than W4A8."""
    K, N = 2048, 256
    w, s, z, g, e2 = _case(fmt, N, K, seed=21)
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=e2)
    sd = s.to(dev)
    for M in (1, 17, 200):
        x = synth.activations(M, K, seed=M, outliers=True)
        exact = _oracle_ref(oracle, x, w, s, z, g, e2)
        a16 = kernels.w4a16_linear(x.to(dev), tiles, sd, None, g, N, weight_is_e2m1=e2).float().cpu().numpy()
        a8 = kernels.w4a8_linear(x.to(dev), tiles, sd, None, g, weight_is_e2m1=e2).float().cpu().numpy()
        d16 = np.linalg.norm(a16 - exact) / np.linalg.norm(exact)
        d8 = np.linalg.norm(a8 - exact) / np.linalg.norm(exact)
        print(f"[w4a16] {fmt} M={M}: |a16-exact| {d16:.3e}  |a8-exact| {d8:.3e}", flush=True)
        assert d16 <= d8


def test_w4a16_dispatch_ledger(kernels, dev):
    eng = pkg("_hip_engage")
    K, N, g = 1024, 128, 128
    w, s, _ = synth.int4_weight(N, K, g, seed=1, asym=False)
    tiles, sd = kernels.repack_w4(w.to(dev)), s.to(dev)
    before = eng.counts()
    kernels.w4a16_linear(synth.activations(2, K, seed=1).to(dev), tiles, sd, None, g, N)
    kernels.w4a16_linear(synth.activations(40, K, seed=1).to(dev), tiles, sd, None, g, N)
    _sync()
    d = eng.counts_delta(before)
    assert d.get("w4a8_mi355x.w4a16_gemv") == 1 and d.get("w4a8_mi355x.w4a16_tiled") == 1


def test_w4a16_refusals(kernels, dev):
    K, N, g = 256, 64, 128
    w, s, _ = synth.int4_weight(N, K, g, seed=2, asym=False)
    tiles, sd = kernels.repack_w4(w.to(dev)), s.to(dev)
    x = synth.activations(2, K, seed=2).to(dev)
    with pytest.raises(AssertionError):
        kernels.w4a16_linear(x, tiles, sd, None, g, N + 16)
    with pytest.raises(TypeError):
        kernels.w4a16_linear(x.float(), tiles, sd, None, g, N)
    with pytest.raises(TypeError):
        kernels.w4a16_act_split(x[:, :100])
