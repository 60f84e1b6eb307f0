"""GPU parity of the dense W4A8 path against the CPU oracle (all through the C ABI).

Bars: fp8 activation codes and scales bit-exact; GEMM outputs within 2e-3 relative L2 of the
oracle's f64 result (the contract), within 5e-4 relative L2 of that result rounded to the output
dtype (what f32 accumulation leaves: see assert_close_to_oracle), with an element-wise structural
guard. Full BASELINE sizes are checked against the oracle where it finishes in seconds (every
decode shape), and through row subsets plus bit-exact row-split invariance for the prefill shapes.
The decode arm is checked for M-invariance: rows[0:m] alone equal the same rows inside a 16-row
call, bit for bit.
"""
import numpy as np
import pytest
import torch

import synth
from conftest import pkg

pytestmark = pytest.mark.gpu

REL_L2 = 2e-3
# Against the oracle rounded to the output dtype, an output differs only where the kernel's f32
# accumulation error moves a value across a rounding boundary of the output dtype. With the
# accumulation error e (relative, about 2^-24 * sqrt(K) for sums of K random-sign terms: under
# 1e-5 at K <= 28672) such a crossing has probability about 2e / ulp and costs one ulp, so the
# relative L2 is about sqrt(2e / ulp) * ulp: 2.5e-4 for bf16 (ulp 2^-8) and 1e-4 for fp16 at the
# largest K. The bar leaves 2x over the bf16 figure.
REL_L2_ROUNDED = 5e-4


def _sync():
    torch.cuda.synchronize()


def assert_close_to_oracle(got: torch.Tensor, ref: np.ndarray, what: str):
    """Contract bar: rel L2 <= 2e-3 against the f64 oracle; on small outputs, where the rounding of
    the exact result to the output dtype alone can reach that (bf16 rounding is about 1.6e-3
    relative L2 on average, more on a few hundred elements), the bar is that rounding's own
    distance plus the kernel bar. Kernel bar: rel L2 <= 5e-4 against the oracle rounded to the
    output dtype (REL_L2_ROUNDED). Structural guard: every element within two output-dtype ulps
    plus 1e-4 of the output's magnitude (the MFMA's fp8 dot product accumulates with slightly less
    than f32 precision, ~1e-5 relative, which shows up only where outputs are small through
    cancellation)."""
    g = got.float().cpu().numpy().astype(np.float64)
    nref = max(np.linalg.norm(ref), 1e-30)
    rel = np.linalg.norm(g - ref) / nref
    dt = torch.bfloat16 if got.dtype == torch.bfloat16 else torch.float16
    rounded = torch.from_numpy(ref).to(dt).double().numpy()
    rel_r = np.linalg.norm(g - rounded) / nref
    bar = max(REL_L2, np.linalg.norm(rounded - ref) / nref + REL_L2_ROUNDED)
    ulp_bits = 7 if got.dtype == torch.bfloat16 else 10
    tol = 2 * np.abs(ref) * 2.0 ** -ulp_bits + 1e-4 * np.abs(ref).max()
    bad = np.abs(g - ref) > tol
    print(f"[parity] {what}: rel L2 {rel:.3e} (vs dtype-rounded oracle {rel_r:.3e}), outliers {int(bad.sum())}",
          flush=True)
    assert rel <= bar, f"{what}: rel L2 {rel:.3e} > {bar:.3e}"
    assert rel_r <= REL_L2_ROUNDED, f"{what}: rel L2 vs the dtype-rounded oracle {rel_r:.3e} > {REL_L2_ROUNDED}"
    assert not bad.any(), f"{what}: {bad.sum()} elements off, worst {np.abs(g - ref)[bad].max():.3e}"
    return rel


# ------------------------------------------------------------------------------- act quant
@pytest.mark.parametrize("dtype,code", [(torch.bfloat16, 0), (torch.float16, 1)])
# 64 rows or more of at most 4096 elements take the one-wave-per-row kernel
@pytest.mark.parametrize("M,K", [(1, 4096), (16, 2560), (7, 14336), (33, 768), (5, 28672), (64, 768), (130, 4096),
                                 (257, 2048), (70, 136)])
def test_act_quant_bit_exact(kernels, oracle, dev, dtype, code, M, K):
    x = synth.activations(M, K, seed=M * 31 + K, outliers=True, dtype=dtype)
    x[0, :] = 0  # scale floor row
    if M > 2:
        x[1, :] = 448.0
        x[2, :] = (torch.linspace(-1e-3, 1e-3, K)).to(dtype)
    q, s = kernels.act_quant(x.to(dev))
    _sync()
    rq, rs = oracle.act_quant(synth.bits16(x), code)
    assert np.array_equal(s.cpu().numpy(), rs), "act scales differ"
    assert np.array_equal(q.cpu().numpy(), rq), f"fp8 codes differ in {(q.cpu().numpy() != rq).sum()} places"


# ------------------------------------------------------------------------------- repack
@pytest.mark.parametrize("e2m1", [False, True])
@pytest.mark.parametrize("N,K", [(32, 256), (48, 160), (16, 2560)])
def test_repack_matches_tile_layout(kernels, dev, e2m1, N, K):
    from test_layout import tile_reference

    w = synth.pack_rows(torch.randint(0, 16, (N, K), generator=synth.gen(N + K), dtype=torch.int32))
    t = kernels.repack_w4(w.to(dev), weight_is_e2m1=e2m1)
    _sync()
    assert tuple(t.shape) == (N // 16, (K + 127) // 128, 1024)
    assert np.array_equal(t.cpu().numpy(), tile_reference(w.numpy(), K, e2m1))


# ------------------------------------------------------------------------------- decode GEMV
def _oracle_dense(oracle, x, w, s, z, g, e2m1=False):
    xq, xs = oracle.act_quant(synth.bits16(x), 0 if x.dtype == torch.bfloat16 else 1)
    return oracle.gemm(xq, xs, w.numpy(), s.numpy(), None if z is None else z.numpy(), g, e2m1)


def test_config1_awq_asym_m16(kernels, oracle, dev):
    """M=16, K=2560, N=9728, AWQ asym int4 g128, scales |N(0,.02)|+1e-4."""
    M, K, N, g = 16, 2560, 9728, 128
    x = synth.activations(M, K, seed=101)
    w, s, z = synth.int4_weight(N, K, g, seed=102, asym=True, scale_floor=1e-4)
    ref = _oracle_dense(oracle, x, w, s, z, g)
    tiles = kernels.repack_w4(w.to(dev))
    out = kernels.w4a8_linear(x.to(dev), tiles, s.to(dev), z.to(dev), g)
    _sync()
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (M, N)
    assert_close_to_oracle(out, ref, "config1")


LLAMA_SHAPES = [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)]  # (K, N)


@pytest.mark.parametrize("K,N", LLAMA_SHAPES)
def test_config2_decode_sweep(kernels, oracle, dev, K, N):
    """GPTQ sym int4 g128 at the four Llama-3-8B layer shapes, M in {1,2,4,8,16},
    activations with 0.1% x50 outlier channels. Every M is checked in full against the oracle."""
    g = 128
    x = synth.activations(16, K, seed=200 + K + N, outliers=True)
    w, s, _ = synth.int4_weight(N, K, g, seed=201 + K + N, asym=False)
    ref = _oracle_dense(oracle, x, w, s, None, g)  # per-row quant: rows of M=16 == rows of any prefix
    tiles = kernels.repack_w4(w.to(dev))
    sd = s.to(dev)
    xd = x.to(dev)
    for M in (1, 2, 4, 8, 16):
        out = kernels.w4a8_linear(xd[:M].contiguous(), tiles, sd, None, g)
        _sync()
        assert_close_to_oracle(out, ref[:M], f"K={K} N={N} M={M}")


M_INV_CASES = [(4096, 6144, 128, "sym"), (4096, 4096, 128, "sym"), (4096, 28672, 128, "sym"), (14336, 4096, 128, "sym"),
               (2560, 9728, 128, "asym"), (2048, 9600, 128, "sym"), (1536, 768, 32, "asym"), (4096, 8192, 32, "e2m1")]


@pytest.mark.parametrize("K,N,g,fmt", M_INV_CASES)
def test_decode_m_invariance(kernels, dev, K, N, g, fmt):
    """The decode arm's self-invariance (tools/quant_m_invariance.py:119-130; the reference records
    worst max|delta| = 0 in _qminv_dense.txt:30-33): rows[0:m] computed alone equal rows[0:m] inside
    a 16-row call, bit for bit, for m = 1..16 -- the Llama-3-8B shapes, configs[0], a 600-strip
    weight whose two-strip grid is small, a sub-tile group and MXFP4. The fused silu arm is held to
    the same."""
    x = synth.activations(16, K, seed=K + N + g, outliers=True).to(dev)
    if fmt == "e2m1":
        w, s = synth.mxfp4_weight(N, K, seed=N + 3)
        z = None
    else:
        w, s, z = synth.int4_weight(N, K, g, seed=N + 3, asym=fmt == "asym", scale_floor=1e-4)
    e2 = fmt == "e2m1"
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=e2)
    sd, zd = s.to(dev), None if z is None else z.to(dev)
    full = kernels.w4a8_linear(x, tiles, sd, zd, g, kernel="decode_gemv", weight_is_e2m1=e2)
    fsilu = kernels.w4a8_linear_silu(x, tiles, sd, zd, g, weight_is_e2m1=e2)
    for m in range(1, 17):
        part = kernels.w4a8_linear(x[:m].contiguous(), tiles, sd, zd, g, kernel="decode_gemv", weight_is_e2m1=e2)
        psilu = kernels.w4a8_linear_silu(x[:m].contiguous(), tiles, sd, zd, g, weight_is_e2m1=e2)
        _sync()
        d = (part.float() - full[:m].float()).abs().max().item()
        assert torch.equal(part, full[:m]), f"K={K} N={N} g={g} {fmt}: rows[0:{m}] differ, max|d| {d:.3e}"
        assert torch.equal(psilu, fsilu[:m]), f"K={K} N={N} g={g} {fmt}: silu rows[0:{m}] differ"


def test_decode_accepts_op_layout_and_explicit_zeros(kernels, oracle, dev):
    """Op-layout weights are repacked on the call; GPTQ's materialised zeros (all 8) give the same
    numbers as the symmetric (None) form."""
    M, K, N, g = 3, 1024, 256, 128
    x = synth.activations(M, K, seed=5)
    w, s, _ = synth.int4_weight(N, K, g, seed=6, asym=False)
    z8 = synth.pack_rows(torch.full((K // g, N), 8, dtype=torch.int32))
    ref = _oracle_dense(oracle, x, w, s, None, g)
    a = kernels.w4a8_linear(x.to(dev), w.to(dev), s.to(dev), None, g)
    b = kernels.w4a8_linear(x.to(dev), w.to(dev), s.to(dev), z8.to(dev), g)
    _sync()
    assert_close_to_oracle(a, ref, "sym None")
    assert_close_to_oracle(b, ref, "sym zeros=8")


@pytest.mark.parametrize("g,asym", [(32, True), (64, False), (256, True)])
def test_decode_group_sizes(kernels, oracle, dev, g, asym):
    M, K, N = 5, 1536, 128
    x = synth.activations(M, K, seed=g)
    w, s, z = synth.int4_weight(N, K, g, seed=g + 1, asym=asym)
    ref = _oracle_dense(oracle, x, w, s, z, g)
    out = kernels.w4a8_linear(x.to(dev), w.to(dev), s.to(dev), None if z is None else z.to(dev), g)
    _sync()
    assert_close_to_oracle(out, ref, f"g={g}")


def test_decode_fp16_activations(kernels, oracle, dev):
    M, K, N, g = 4, 2048, 256, 128
    x = synth.activations(M, K, seed=77, dtype=torch.float16)
    w, s, z = synth.int4_weight(N, K, g, seed=78, asym=True)
    ref = _oracle_dense(oracle, x, w, s, z, g)
    out = kernels.w4a8_linear(x.to(dev), w.to(dev), s.to(dev), z.to(dev), g)
    _sync()
    assert out.dtype == torch.float16
    assert_close_to_oracle(out, ref, "fp16")


# ------------------------------------------------------------------------------- prefill GEMM
@pytest.mark.parametrize("K,N", LLAMA_SHAPES)
def test_config3_prefill(kernels, oracle, dev, K, N):
    """the same shapes at M in {512, 2048, 8192} on the MFMA arm. A row subset
    of each run is checked against the oracle; every row must equal the row computed alone
    (bit-exact row-split / M-invariance)."""
    g = 128
    w, s, _ = synth.int4_weight(N, K, g, seed=300 + K + N, asym=False)
    tiles = kernels.repack_w4(w.to(dev))
    sd = s.to(dev)
    for M in (512, 2048, 8192):
        x = synth.activations(M, K, seed=301 + M, outliers=True)
        xd = x.to(dev)
        out = kernels.w4a8_linear(xd, tiles, sd, None, g)
        rows = torch.tensor(sorted({0, 1, 17, M // 3, M // 2 + 5, M - 2, M - 1}))
        part = kernels.w4a8_linear(xd[rows].contiguous(), tiles, sd, None, g, kernel="wmma_tiled_tuned")
        _sync()
        assert torch.equal(out[rows.to(dev)], part), f"row-split invariance broken at M={M}"
        ref = _oracle_dense(oracle, x[rows], w, s, None, g)
        assert_close_to_oracle(part, ref, f"prefill K={K} N={N} M={M}")


def test_prefill_asym_ragged(kernels, oracle, dev):
    """Zero points, M not a multiple of the tile, K not a multiple of 128, N not a multiple of 128."""
    M, K, N, g = 77, 1184, 208, 32
    x = synth.activations(M, K, seed=9)
    w, s, z = synth.int4_weight(N, K, g, seed=10, asym=True)
    ref = _oracle_dense(oracle, x, w, s, z, g)
    out = kernels.w4a8_linear(x.to(dev), w.to(dev), s.to(dev), z.to(dev), g)
    _sync()
    assert_close_to_oracle(out, ref, "prefill ragged")


def test_decode_and_prefill_arms_agree(kernels, oracle, dev):
    M, K, N, g = 16, 4096, 1024, 128
    x = synth.activations(M, K, seed=41)
    w, s, _ = synth.int4_weight(N, K, g, seed=42, asym=False)
    tiles = kernels.repack_w4(w.to(dev))
    a = kernels.w4a8_linear(x.to(dev), tiles, s.to(dev), None, g, kernel="decode_gemv")
    b = kernels.w4a8_linear(x.to(dev), tiles, s.to(dev), None, g, kernel="wmma_tiled_tuned")
    _sync()
    ref = _oracle_dense(oracle, x, w, s, None, g)
    assert_close_to_oracle(a, ref, "decode arm")
    assert_close_to_oracle(b, ref, "prefill arm")


# ------------------------------------------------------------------------------- MXFP4
@pytest.mark.parametrize("K,N", [(8192, 28672), (28672, 8192)])
def test_config5_mxfp4(kernels, oracle, dev, K, N):
    """e2m1 codes, E8M0 block-32 scales (exponents in [-8, 0]), M in {1, 16, 4096}."""
    w, s8 = synth.mxfp4_weight(N, K, seed=500 + K)
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=True)
    sd = s8.to(dev)
    x = synth.activations(16, K, seed=501 + K)
    ref = _oracle_dense(oracle, x, w, s8, None, 32, e2m1=True)
    for M in (1, 16):
        out = kernels.w4a8_linear(x[:M].contiguous().to(dev), tiles, sd, None, 32, weight_is_e2m1=True)
        _sync()
        assert_close_to_oracle(out, ref[:M], f"mxfp4 K={K} N={N} M={M}")
    M = 4096
    xb = synth.activations(M, K, seed=502 + K)
    xd = xb.to(dev)
    out = kernels.w4a8_linear(xd, tiles, sd, None, 32, weight_is_e2m1=True)
    rows = torch.tensor([0, 5, 1000, 2047, 4095])
    part = kernels.w4a8_linear(xd[rows].contiguous(), tiles, sd, None, 32, kernel="wmma_tiled_tuned",
                               weight_is_e2m1=True)
    _sync()
    assert torch.equal(out[rows.to(dev)], part)
    assert_close_to_oracle(part, _oracle_dense(oracle, xb[rows], w, s8, None, 32, e2m1=True), "mxfp4 M=4096")


def test_e2m1_with_fp16_group_scales(kernels, oracle, dev):
    """The fp16-folded MXFP4 scale form (python/minisgl/quant/mxfp4.py:71-97) on both arms."""
    K, N = 1024, 256
    w, s8 = synth.mxfp4_weight(N, K, seed=61)
    s16 = torch.pow(2.0, s8.float() - 127).to(torch.float16)
    for M in (3, 40):
        x = synth.activations(M, K, seed=62 + M)
        ref = _oracle_dense(oracle, x, w, s8, None, 32, e2m1=True)
        out = kernels.w4a8_linear(x.to(dev), w.to(dev), s16.to(dev), None, 32, weight_is_e2m1=True)
        _sync()
        assert_close_to_oracle(out, ref, f"e2m1 fp16-scale M={M}")


# ------------------------------------------------------------------------------- fused silu
SILU_SHAPES = [(1, 256, 512, 128), (2, 512, 1024, 128), (4, 768, 2048, 128), (1, 512, 1536, 128), (1, 384, 1024, 32)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("fmt", ["sym", "asym", "e2m1"])
def test_fused_silu_bit_exact(kernels, dev, dtype, fmt):
    """tools/w4a8_gemm_silu_parity.py: fused == unfused decode GEMV + round-silu-round-mul replica,
    bit for bit."""
    for (M, inter, K, g) in SILU_SHAPES:
        N = 2 * inter
        x = (synth.activations(M, K, seed=M + inter + K, dtype=torch.float32) * 0.3).to(dtype).to(dev)
        if fmt == "e2m1":
            if g != 32:
                continue
            w, s = synth.mxfp4_weight(N, K, seed=inter)
            z = None
        else:
            w, s, z = synth.int4_weight(N, K, g, seed=inter, asym=fmt == "asym", scale_floor=0.001)
        w, s = w.to(dev), s.to(dev)
        z = None if z is None else z.to(dev)
        e2 = fmt == "e2m1"
        out1 = kernels.w4a8_linear(x, w, s, z, g, kernel="decode_gemv", weight_is_e2m1=e2)
        gh, uh = out1[:, :inter], out1[:, inter:]
        ref = (gh.float() / (1.0 + torch.exp(-gh.float()))).to(dtype) * uh
        fused = kernels.w4a8_linear_silu(x, w, s, z, g, weight_is_e2m1=e2)
        _sync()
        assert torch.equal(fused, ref), f"{fmt} {dtype} M={M} inter={inter} K={K} g={g}: max " \
                                        f"{(fused.float() - ref.float()).abs().max().item():.3e}"


# ------------------------------------------------------------------------------- producer pair
@pytest.mark.parametrize("M", [1, 17, 129])
def test_producer_pair_bit_identical(kernels, dev, M):
    K, N, g = 2048, 512, 128
    x = synth.activations(M, K, seed=M).to(dev)
    w, s, _ = synth.int4_weight(N, K, g, seed=M + 1, asym=False)
    tiles, sd = kernels.repack_w4(w.to(dev)), s.to(dev)
    q, sc = kernels.act_quant(x)
    base = kernels.w4a8_linear(x, tiles, sd, None, g)
    pre = kernels.w4a8_linear(x, tiles, sd, None, g, x_fp8=q, act_scales=sc)
    pre8 = kernels.w4a8_linear(x, tiles, sd, None, g, x_fp8=q.view(torch.float8_e4m3fn), act_scales=sc)
    _sync()
    assert torch.equal(base, pre) and torch.equal(base, pre8)


def _row_major_gemm(q, sc, tiles, s, z, g, N, K, e2, out_dtype):
    """The prefill GEMM on row-major codes: the C ABI's w4a8_gemm with no workspace (no rewrite into
    the operand order), so the kernel computes the row-sum seeds itself."""
    abi = pkg("_abi")
    lib = abi.load()
    y = torch.empty((q.shape[0], N), dtype=out_dtype, device=q.device)
    sfmt = abi.SCALE_F16 if s.dtype == torch.float16 else abi.SCALE_E8M0
    odt = abi.BF16 if out_dtype == torch.bfloat16 else abi.F16
    abi.check(lib.w4a8_gemm(abi.ptr(q), K, abi.ptr(sc), q.shape[0], abi.ptr(tiles), N, K, abi.ptr(s), sfmt,
                            abi.ptr(z), abi.W_E2M1 if e2 else abi.W_INT4, g, abi.ptr(y), odt, N, 0, None, 0,
                            abi.KERNEL_PREFILL, abi.stream_of(q)), "w4a8_gemm")
    return y


@pytest.mark.parametrize("fmt,M,K,N", [("sym", 2048, 4096, 28672), ("sym", 1100, 1024, 16400), ("sym16", 1030, 2048, 16384),
                                        ("sym", 1030, 1024, 4096), ("sym", 1100, 5120, 2048), ("sym", 1024, 768, 2048),
                                        ("sym", 300, 1024, 512), ("asym", 1100, 1024, 16384), ("mxfp4", 1024, 4096, 1024),
                                        ("mxfp4", 1100, 2048, 4096), ("mxfp4", 1024, 1024, 16384)])
def test_prefill_tiled_quant_matches_row_major(kernels, dev, fmt, M, K, N):
    """Symmetric int4 and MXFP4 prefill calls of 1024+ rows on 2048+ output channels that quantize x
    themselves write the codes in the GEMM's operand order (act_quant_tiled_lds_kernel for K <= 4096,
    the two-pass act_quant_tiled_kernel above: K=5120 here), with the row-sum seeds the int4 GEMM
    reads instead of computing. The same bits as the GEMM on row-major codes (w4a8_gemm with no
    workspace), and as the producer pair (rewritten into the operand order on 16384+ channels); also
    on a ragged 1025-strip weight and the formats that stay row-major (zero points, narrow MXFP4)."""
    x = synth.activations(M, K, seed=M + K, outliers=True).to(dev)
    if fmt == "sym16":  # fp16 activations (scale rows, codes and seeds from fp16 values)
        x = x.to(torch.float16)
    if fmt == "mxfp4":
        w, s = synth.mxfp4_weight(N, K, seed=N + 1)
        z, g, e2 = None, 32, True
    else:
        w, s, z = synth.int4_weight(N, K, 128, seed=N + 1, asym=fmt == "asym", scale_floor=1e-4)
        g, e2 = 128, False
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=e2)
    sd, zd = s.to(dev), None if z is None else z.to(dev)
    q, sc = kernels.act_quant(x)
    base = kernels.w4a8_linear(x, tiles, sd, zd, g, weight_is_e2m1=e2)
    pre = kernels.w4a8_linear(x, tiles, sd, zd, g, weight_is_e2m1=e2, x_fp8=q, act_scales=sc)
    rm = _row_major_gemm(q, sc, tiles, sd, zd, g, N, K, e2, x.dtype)
    _sync()
    assert torch.equal(base, pre), f"{fmt} M={M}: max {(base.float() - pre.float()).abs().max().item():.3e}"
    assert torch.equal(base, rm), f"{fmt} M={M}: max {(base.float() - rm.float()).abs().max().item():.3e}"


def test_dispatch_ledger_records_arms(kernels, dev):
    eng = pkg("_hip_engage")
    K, N, g = 1024, 128, 128
    w, s, _ = synth.int4_weight(N, K, g, seed=1, asym=False)
    tiles, sd = kernels.repack_w4(w.to(dev)), s.to(dev)
    before = eng.counts()
    kernels.w4a8_linear(synth.activations(2, K, seed=1).to(dev), tiles, sd, None, g)
    kernels.w4a8_linear(synth.activations(40, K, seed=1).to(dev), tiles, sd, None, g)
    _sync()
    d = eng.counts_delta(before)
    assert d.get("w4a8_mi355x.gemm(decode_gemv)") == 1 and d.get("w4a8_mi355x.gemm(wmma_tiled_tuned)") == 1


# ------------------------------------------------------------------------------- edge shapes
@pytest.mark.parametrize("fmt,g", [("sym", 32), ("asym", 64), ("mxfp4", 32), ("nvfp4", 16)])
@pytest.mark.parametrize("M,K,N", [(17, 160, 16), (40, 2592, 48), (300, 1088, 144), (5, 96, 32)])
def test_edge_shapes(kernels, oracle, dev, fmt, g, M, K, N):
    """K that is not a multiple of 128 (the tile's zero padding, the per-wave prefill kernel), one
    strip (N=16), row counts on both arms, every weight format; against the oracle."""
    if K % g:
        pytest.skip("group does not divide K")
    if fmt in ("sym", "asym"):
        w, s, z = synth.int4_weight(N, K, g, seed=M + K, asym=fmt == "asym", scale_floor=1e-4)
        e2, nv = False, False
    elif fmt == "mxfp4":
        w, s = synth.mxfp4_weight(N, K, seed=M + K)
        z, e2, nv = None, True, False
    else:
        w, s, z = synth.nvfp4_weight(N, K, seed=M + K)
        e2, nv = True, True
    x = synth.activations(M, K, seed=M)
    xq, xs = oracle.act_quant(synth.bits16(x), 0)
    sv = s.view(torch.uint8).numpy() if nv else s.numpy()
    ref = oracle.gemm(xq, xs, w.numpy(), sv, None if z is None else z.numpy(), g, e2, nv)
    tiles = kernels.repack_w4(w.to(dev), weight_is_e2m1=e2)
    out = kernels.w4a8_linear(x.to(dev), tiles, s.to(dev), None if z is None else z.to(dev), g, weight_is_e2m1=e2)
    _sync()
    assert tuple(out.shape) == (M, N)
    assert_close_to_oracle(out, ref, f"{fmt} g={g} M={M} K={K} N={N}")


def test_empty_batch(kernels, dev):
    """M = 0 returns an empty (0, N) result on both arms and the fused silu arm, without a launch
    error."""
    K, N, g = 512, 64, 128
    w, s, _ = synth.int4_weight(N, K, g, seed=3, asym=False)
    tiles, sd = kernels.repack_w4(w.to(dev)), s.to(dev)
    x = torch.empty((0, K), dtype=torch.bfloat16, device=dev)
    for kern in (None, "decode_gemv", "wmma_tiled_tuned"):
        out = kernels.w4a8_linear(x, tiles, sd, None, g, kernel=kern)
        assert tuple(out.shape) == (0, N)
    assert tuple(kernels.w4a8_linear_silu(x, tiles, sd, None, g).shape) == (0, N // 2)
    _sync()
