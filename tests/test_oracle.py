"""Pins the CPU oracle (oracle/w4a8_oracle.c) before anything is checked against it.

Each check is chosen so a plausible slip (wrong rounding, dropped term, transposed operand,
off-by-one zero point, wrong tie rule) fails: library routines (torch's float8_e4m3fn cast),
closed forms, the reference's own test vectors and worked examples, and brute force on tiny inputs.
"""
import numpy as np
import pytest
import torch

import synth


# ------------------------------------------------------------------------------------ e4m3 codec
def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_decode_all_codes_matches_torch(oracle):
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy().astype(np.float64)
    got = oracle.e4m3_decode(codes)
    c_got = np.array([oracle.lib().w4o_e4m3_to_f32(int(c)) for c in codes], dtype=np.float64)
    nan = np.isnan(ref)
    assert set(np.nonzero(nan)[0]) == {0x7F, 0xFF}
    assert np.array_equal(np.isnan(got), nan) and np.array_equal(np.isnan(c_got), nan)
    assert np.array_equal(got[~nan], ref[~nan]) and np.array_equal(c_got[~nan], ref[~nan])


def _e4m3_probe_values(n_random: int = 20000) -> np.ndarray:
    pos = np.array([v for v in oracle_decode_positive()], dtype=np.float64)
    mids = 0.5 * (pos[:-1] + pos[1:])
    mids32 = mids.astype(np.float32)
    xs = [pos.astype(np.float32), mids32, np.nextafter(mids32, np.float32(1e9)), np.nextafter(mids32, np.float32(-1e9)),
          np.array([448.0, 449.0, 463.99, 2.0 ** -10, 2.0 ** -11, 1.5 * 2.0 ** -10, 1e-30, 0.0], dtype=np.float32)]
    rng = np.random.default_rng(0)
    r = (1.0 + rng.random(n_random)) * 2.0 ** rng.integers(-14, 9, n_random)
    xs.append(r[r < 448].astype(np.float32))
    v = np.concatenate(xs)
    return np.concatenate([v, -v])


def oracle_decode_positive():
    for c in range(0x7F):
        e, m = c >> 3, c & 7
        yield m * 2.0 ** -9 if e == 0 else (8 + m) * 2.0 ** (e - 10)


def test_e4m3_encode_matches_torch_rne(oracle):
    x = _e4m3_probe_values()
    got = oracle.e4m3_encode(x)
    assert np.array_equal(got, _torch_e4m3(x))


def test_e4m3_encode_ties_to_even(oracle):
    # 1.0625 lies exactly between 1.0 (mantissa 000) and 1.125 (001): even -> 1.0
    # 1.1875 between 1.125 (001) and 1.25 (010): even -> 1.25
    assert oracle.e4m3_decode(oracle.e4m3_encode(np.array([1.0625], np.float32)))[0] == 1.0
    assert oracle.e4m3_decode(oracle.e4m3_encode(np.array([1.1875], np.float32)))[0] == 1.25
    # subnormal tie: 2^-10 is halfway between 0 and 2^-9 -> 0
    assert oracle.e4m3_encode(np.array([2.0 ** -10], np.float32))[0] == 0


# ------------------------------------------------------------------------------------ act quant
def _act_quant_restated(x: torch.Tensor):
    """amax/448 floored at 1e-8, f32 reciprocal, f32 multiply, torch RNE cast."""
    xf = x.float().numpy()
    amax = np.abs(xf).max(axis=1).astype(np.float32)
    s = (amax / np.float32(448.0)).astype(np.float32)
    s = np.where(s < np.float32(1e-8), np.float32(1e-8), s).astype(np.float32)
    inv = (np.float32(1.0) / s).astype(np.float32)
    t = (xf * inv[:, None]).astype(np.float32)
    return _torch_e4m3(t), s


@pytest.mark.parametrize("dtype,code", [(torch.bfloat16, 0), (torch.float16, 1)])
def test_act_quant_matches_restatement(oracle, dtype, code):
    x = synth.activations(8, 512, seed=3, outliers=True, dtype=dtype)
    special = torch.zeros(6, 512, dtype=dtype)
    special[1, 5] = 3.0                    # single nonzero
    special[2, :] = 448.0                  # amax exactly 448 -> scale 1.0
    special[2, 7] = -448.0
    special[3, :] = torch.linspace(-1e-6, 1e-6, 512).to(dtype)  # scale floor active
    special[4, ::2] = 1.0
    special[4, 1::2] = -0.5
    special[5, :] = torch.randn(512, generator=synth.gen(9)).to(dtype) * 1e4
    x = torch.cat([x, special])
    q, s = oracle.act_quant(synth.bits16(x), code)
    rq, rs = _act_quant_restated(x)
    assert np.array_equal(s, rs)
    assert np.array_equal(q, rq)
    assert q[8].max() == 0 and s[8] == np.float32(1e-8)       # all-zero row
    assert s[10] == np.float32(1.0)


# ------------------------------------------------------------------------------------ decode tables
def test_e2m1_lut_is_reference_table(oracle):
    # python/minisgl/quant/mxfp4.py:37-38
    ref = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    got = [oracle.lib().w4o_e4m3_to_f32(0) * 0 + float(v) for v in oracle.E2M1_LUT]
    assert got == ref
    # and the C table the GEMM uses: dequantize one row with unit E8M0 scales (code 127)
    codes = torch.arange(16, dtype=torch.int32).repeat(2).reshape(1, 32)
    w = synth.pack_rows(codes).numpy()
    sc = np.full((1, 1), 127, dtype=np.uint8)
    deq = oracle.dequant(np.repeat(w, 16, 0), np.repeat(sc, 16, 1), None, 32, e2m1=True)[0]
    assert deq.tolist() == ref + ref


def test_e8m0_decode_is_shift(oracle):
    """tests/mxfp4_e8m0_test.py:23-42: value = bitcast(s << 23) for s in [1, 254], s=0 -> 2^-127."""
    s = np.arange(0, 255, dtype=np.uint8)
    N = 16
    codes = np.full((N, 32), 2, dtype=np.int32)  # e2m1 code 2 = 1.0
    w = synth.pack_rows(torch.from_numpy(codes)).numpy()
    got = []
    for sv in s:
        sc = np.full((1, N), sv, dtype=np.uint8)
        got.append(oracle.dequant(w, sc, None, 32, e2m1=True)[0, 0])
    shift = (s.astype(np.uint32) << 23).view(np.float32).astype(np.float64)
    shift[0] = 2.0 ** -127
    assert np.array_equal(np.array(got), shift)


# ------------------------------------------------------------------------------------ GEMM
def _np_unpack(w: np.ndarray) -> np.ndarray:
    sh = np.arange(0, 32, 4, dtype=np.uint32)
    u = (w.astype(np.uint32)[..., None] >> sh) & 15
    return u.reshape(*w.shape[:-1], w.shape[-1] * 8).astype(np.int64)


def _np_gemm(xq, xs, w, scales, zeros, group, e2m1):
    """Independent dequantize-then-matmul: (N,K) codes -> values; per-channel zero unpack along N."""
    codes = _np_unpack(w)
    N, K = codes.shape
    if e2m1:
        wv = oracle_e2m1()[codes]
    else:
        if zeros is None:
            z = np.full((K // group, N), 8)
        else:
            z = _np_unpack(zeros)  # (G, N)
        wv = codes - np.repeat(z, group, axis=0).T
    if scales.dtype == np.uint8:
        sc = 2.0 ** (scales.astype(np.float64) - 127)
    else:
        sc = scales.astype(np.float64)
    wd = wv * np.repeat(sc, group, axis=0).T
    import oracle as o

    xv = o.e4m3_decode(xq)
    return (xv @ wd.T) * xs.astype(np.float64)[:, None]


def oracle_e2m1():
    import oracle as o

    return o.E2M1_LUT


@pytest.mark.parametrize("group,asym,e2m1,sfmt", [(128, False, False, "f16"), (128, True, False, "f16"),
                                                   (64, True, False, "f16"), (32, False, False, "f16"),
                                                   (32, False, True, "e8m0"), (32, False, True, "f16")])
def test_gemm_brute_force(oracle, group, asym, e2m1, sfmt):
    M, N, K = 3, 16, 256
    x = synth.activations(M, K, seed=11)
    xq, xs = oracle.act_quant(synth.bits16(x), 0)
    if e2m1:
        w, s8 = synth.mxfp4_weight(N, K, seed=12)
        w = w.numpy()
        scales = s8.numpy() if sfmt == "e8m0" else (2.0 ** (s8.numpy().astype(np.float64) - 127)).astype(np.float16)
        if sfmt == "f16" and group != 32:
            pytest.skip("fp16-scaled e2m1 uses the 32-block")
        zeros = None
    else:
        w, s, z = synth.int4_weight(N, K, group, seed=12, asym=asym)
        w, scales, zeros = w.numpy(), s.numpy(), None if z is None else z.numpy()
    got = oracle.gemm(xq, xs, w, scales, zeros, group, e2m1)
    ref = _np_gemm(xq, xs, w, scales, zeros, group, e2m1)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_gemm_row_split_and_linearity(oracle):
    M, N, K = 6, 32, 384
    x = synth.activations(M, K, seed=21, outliers=True)
    xq, xs = oracle.act_quant(synth.bits16(x), 0)
    w, s, z = synth.int4_weight(N, K, 128, seed=22, asym=True)
    w, s, z = w.numpy(), s.numpy(), z.numpy()
    full = oracle.gemm(xq, xs, w, s, z, 128)
    part = oracle.gemm(xq[2:5], xs[2:5], w, s, z, 128)
    assert np.array_equal(full[2:5], part)
    # doubling every group scale (exact in fp16) doubles the output exactly
    two = oracle.gemm(xq, xs, w, (s.astype(np.float32) * 2).astype(np.float16), z, 128)
    assert np.array_equal(two, 2 * full)


# ------------------------------------------------------------------------------------ MoE
def test_moe_align_worked_example(oracle):
    """python/minisgl/moe/fused.py:80-97: topk_ids [[2,3,4],[1,2,4],[1,3,4],[1,2,3]], block 4 ->
    sorted [3,6,9,12, 0,4,10,12, 1,7,11,12, 2,5,8,12] (experts 1..4; expert 0 empty)."""
    ids = np.array([[2, 3, 4], [1, 2, 4], [1, 3, 4], [1, 2, 3]], dtype=np.int32)
    sorted_ids, expert_ids, ntp, inv = oracle.moe_align(ids, 5, 4)
    assert ntp == 16
    assert sorted_ids[:16].tolist() == [3, 6, 9, 12, 0, 4, 10, 12, 1, 7, 11, 12, 2, 5, 8, 12]
    assert (sorted_ids[16:] == 12).all()
    assert expert_ids[:4].tolist() == [1, 2, 3, 4] and (expert_ids[4:] == 4).all()
    for slot, pos in enumerate(inv):
        assert sorted_ids[pos] == slot


def test_moe_align_dropped_slots_are_an_extra_last_expert(oracle):
    """Ids outside [0, E) are dropped: the layout of experts 0..E-1 equals that of the same route
    with the dropped slots sent to an extra expert E (which sorts last), ntp ends where that extra
    expert would start, and a dropped slot's inverse position is -1."""
    rng = np.random.default_rng(5)
    E, bm = 12, 16
    ids = rng.integers(0, E, size=(300, 4)).astype(np.int32)
    drop = rng.random(ids.shape) < 0.2
    ids_d = np.where(drop, np.where(rng.random(ids.shape) < 0.5, -1, E + 3), ids).astype(np.int32)
    s, e, ntp, inv = oracle.moe_align(ids_d, E, bm)
    s2, e2, ntp2, inv2 = oracle.moe_align(np.where(drop, E, ids).astype(np.int32), E + 1, bm)
    assert ntp < ntp2 and np.array_equal(s[:ntp], s2[:ntp]) and (s[ntp:] == ids.size).all()
    assert np.array_equal(e[: ntp // bm], e2[: ntp // bm]) and (e[ntp // bm:] == E - 1).all()
    assert np.array_equal(inv[~drop.ravel()], inv2[~drop.ravel()]) and (inv[drop.ravel()] == -1).all()


def test_moe_align_matches_stable_sort(oracle):
    rng = np.random.default_rng(5)
    for T, E, k, bm in [(1, 128, 8, 16), (16, 128, 8, 16), (37, 16, 4, 32), (300, 128, 8, 64)]:
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
        sorted_ids, expert_ids, ntp, inv = oracle.moe_align(ids, E, bm)
        flat = ids.ravel()
        order = np.argsort(flat, kind="stable")
        cnt = np.bincount(flat, minlength=E)
        pad = (cnt + bm - 1) // bm * bm
        start = np.concatenate([[0], np.cumsum(pad)[:-1]])
        exp = np.full(flat.size + (E + 1) * (bm - 1), flat.size, dtype=np.int64)
        fill = np.zeros(E, dtype=np.int64)
        for slot in order:
            e = flat[slot]
            exp[start[e] + fill[e]] = slot
            fill[e] += 1
        assert ntp == pad.sum()
        assert np.array_equal(sorted_ids, exp)
        blk_owner = np.searchsorted(np.cumsum(pad // bm), np.arange(expert_ids.size), side="right")
        assert np.array_equal(expert_ids, np.minimum(blk_owner, E - 1))


def test_moe_route_ties_keep_lower_index(oracle):
    """python/minisgl/layers/moe.py:1218-1227: exact ties at the k-th boundary keep the lower index."""
    logits = np.zeros((2, 8), dtype=np.float32)
    logits[0] = [0.5, 1.0, 1.0, 1.0, -1.0, 1.0, 0.0, 2.0]  # 2.0 then four tied 1.0s; top-3 -> 7, 1, 2
    logits[1] = [3.0, 3.0, 3.0, 3.0, 3.0, 3.0, 3.0, 3.0]
    tw, ids = oracle.moe_route(logits, 3, renormalize=True)
    assert ids[0].tolist() == [7, 1, 2]
    assert ids[1].tolist() == [0, 1, 2]
    np.testing.assert_allclose(tw[1], [1 / 3] * 3, rtol=1e-6)
    p = np.exp(logits[0] - logits[0].max())
    p /= p.sum()
    sel = p[[7, 1, 2]]
    np.testing.assert_allclose(tw[0], sel / (sel.sum() + 1e-8), rtol=1e-6)


def test_moe_route_matches_torch_topk_without_ties(oracle):
    lg = synth.router_logits(64, 128, seed=4, dtype=torch.float32).numpy()
    tw, ids = oracle.moe_route(lg, 8, renormalize=True)
    p = torch.softmax(torch.from_numpy(lg).double(), -1)
    rw, ri = torch.topk(p, 8, dim=-1)
    assert np.array_equal(ids, ri.numpy())
    rw = rw / (rw.sum(-1, keepdim=True) + 1e-8)
    np.testing.assert_allclose(tw, rw.numpy(), rtol=1e-6)


def test_silu_mul_replica(oracle):
    """tools/w4a8_gemm_silu_parity.py:52-54 in torch (CPU) vs the C replica."""
    rng = np.random.default_rng(1)
    g = rng.standard_normal(2000) * 4
    u = rng.standard_normal(2000) * 4
    gb = torch.tensor(g, dtype=torch.float32).to(torch.bfloat16)
    ub = torch.tensor(u, dtype=torch.float32).to(torch.bfloat16)
    silu_h = (gb.float() / (1.0 + torch.exp(-gb.float()))).to(torch.bfloat16)
    ref = (silu_h * ub).view(torch.int16).numpy().view(np.uint16)
    got = np.array([oracle.silu_mul(a, b, 0) for a, b in zip(g, u)], dtype=np.uint16)
    # the f32 exp of two libms may differ by an ulp; after two bf16 roundings they almost always agree
    diff = np.abs(oracle.bf16_to_f32(got).astype(np.float64) - oracle.bf16_to_f32(ref).astype(np.float64))
    ulp = np.abs(oracle.bf16_to_f32(ref)).astype(np.float64) * 2.0 ** -7 + 1e-30
    assert (diff <= ulp).all()
    assert (got == ref).mean() > 0.99


def test_moe_forward_matches_composition(oracle):
    """The fused oracle MoE == route -> align -> per-slot gemm1 -> silu -> act-quant -> gemm2 -> combine,
    with each slot's gemm2 row entering the combine unrounded, or (round_y2) rounded to x's dtype."""
    T, H, I, E, k, g = 5, 256, 128, 8, 2, 128
    x = synth.activations(T, H, seed=31)
    w13, s13, _ = synth.int4_weight(2 * I, H, g, seed=32, asym=False, E=E)
    w2, s2, _ = synth.int4_weight(H, I, g, seed=33, asym=False, E=E)
    w13, s13, w2, s2 = w13.numpy(), s13.numpy(), w2.numpy(), s2.numpy()
    lg = synth.router_logits(T, E, seed=34, dtype=torch.float32).numpy()
    tw, ids = oracle.moe_route(lg, k)
    sorted_ids, expert_ids, ntp, inv = oracle.moe_align(ids, E, 16)
    out = oracle.moe_forward(synth.bits16(x), 0, tw, sorted_ids, expert_ids, ntp, 16, k, w13, s13, None, w2, s2, None)
    xq, xs = oracle.act_quant(synth.bits16(x), 0)
    ref = np.zeros((T, H))
    ref_r = np.zeros((T, H))
    for t in range(T):
        for j in range(k):
            e = ids[t, j]
            h = oracle.gemm(xq[t:t + 1], xs[t:t + 1], w13[e], s13[e], None, g)[0]
            b2 = np.array([oracle.silu_mul(h[i], h[I + i], 0) for i in range(I)], dtype=np.uint16)
            q2, s2v = oracle.act_quant(b2[None, :], 0)
            y = oracle.gemm(q2, s2v, w2[e], s2[e], None, g)[0]
            ref[t] += tw[t, j] * y
            # the unfused contract: the slot's gemm2 row reaches the combine in x's dtype (torch's
            # RNE f32 -> bf16 cast, independent of the oracle's own rounding helpers)
            yr = torch.from_numpy(y.astype(np.float32)).to(torch.bfloat16).double().numpy()
            ref_r[t] += tw[t, j] * yr
    np.testing.assert_allclose(out, ref, rtol=1e-9, atol=1e-9)
    out_r = oracle.moe_forward(synth.bits16(x), 0, tw, sorted_ids, expert_ids, ntp, 16, k, w13, s13, None, w2, s2, None,
                               round_y2=True)
    np.testing.assert_allclose(out_r, ref_r, rtol=1e-9, atol=1e-9)
    assert not np.allclose(out_r, out, rtol=1e-6, atol=0)  # the rounding is really applied


# ------------------------------------------------------------------------------- RMSNorm producer
def _bits(t):
    return synth.bits16(t)


def _from_bits(b, dtype):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(dtype)


@pytest.mark.parametrize("dtype,code", [(torch.bfloat16, 0), (torch.float16, 1)])
@pytest.mark.parametrize("K", [2048, 2816, 5120, 13, 8])
def test_rms_norm_matches_torch_decomposition(oracle, dtype, code, K):
    """The oracle's norm against the reference's own torch decomposition (python/minisgl/layers/
    norm.py:19-24: f32 mean of squares, rsqrt, round to dtype, times the gain in dtype), including
    plus_one and the unweighted form. The two sum the squares in different orders, so a last-bit
    difference in the mean may move a rounding: at most 1 output ulp, on a small share of elements."""
    if K % 8:
        K = 8 * K  # rows are whole 16-byte chunks on the device; the oracle itself takes any K
    g = torch.Generator().manual_seed(K + code)
    M = 6
    x = (torch.randn(M, K, generator=g) * 0.7).to(dtype)
    x[0] = 0  # an all-zero row: rstd = 1/sqrt(eps), output zero
    w = (torch.randn(K, generator=g) * 0.1 + 1.0).to(dtype)
    for weight, plus_one in ((w, False), (w - 1.0, True), (None, False)):
        o, _ = oracle.rms_norm(_bits(x), None if weight is None else _bits(weight.to(dtype)), 1e-6, code, plus_one)
        xf = x.float()
        var = xf.pow(2).mean(dim=-1, keepdim=True)
        ref = (xf * torch.rsqrt(var + 1e-6)).to(dtype)
        if weight is not None:
            ref = ref * (weight.to(dtype) + 1.0) if plus_one else ref * weight.to(dtype)
        got = _from_bits(o, dtype)
        diff = (got.view(torch.int16).int() - ref.view(torch.int16).int()).abs()
        assert int(diff.max()) <= 1, f"K={K} plus_one={plus_one}: {int(diff.max())} ulp"
        assert float((diff > 0).float().mean()) < 0.01
        assert torch.equal(got[0], torch.zeros(K, dtype=dtype))


def test_rms_norm_add_residual_is_dtype_sum(oracle):
    """rms_norm_add: residual <- x + residual with one rounding to the dtype (torch's bf16 add), and
    the norm runs over that sum (python/minisgl/layers/norm.py:134-138)."""
    g = torch.Generator().manual_seed(5)
    for dtype, code in ((torch.bfloat16, 0), (torch.float16, 1)):
        x = torch.randn(4, 2048, generator=g).to(dtype)
        r = torch.randn(4, 2048, generator=g).to(dtype)
        w = (torch.randn(2048, generator=g) * 0.1 + 1).to(dtype)
        o, nr = oracle.rms_norm(_bits(x), _bits(w), 1e-5, code, False, residual_bits=_bits(r))
        assert torch.equal(_from_bits(nr, dtype), x + r)
        o2, _ = oracle.rms_norm(_bits(x + r), _bits(w), 1e-5, code, False)
        assert np.array_equal(o, o2)


# ------------------------------------------------------------------------------- w4a16 split
def _split_recon(codes: np.ndarray, scales: np.ndarray, T: int) -> np.ndarray:
    dec = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    v = (dec * scales.astype(np.float64)[:, None]).reshape(-1, T, codes.shape[1]).sum(axis=1)
    return v


@pytest.mark.parametrize("dtype,code,T", [(torch.bfloat16, 0, 2), (torch.float16, 1, 3)])
def test_w4a16_split_is_exact(oracle, dtype, code, T):
    """x == sum_t scale_t * e4m3(code_t) exactly, on random rows with outliers and on edge rows
    (all zero, one nonzero, amax exactly 448 * 2^j and just above, mixed binades)."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(6, 512, generator=g) * torch.logspace(-3, 3, 6)[:, None]
    x[0] = 0.0
    x[1] = 0.0
    x[1, 17] = -3.25
    x[2, :] = torch.linspace(-448.0, 448.0, 512)
    x[3, :] = torch.linspace(-1.0, 1.0, 512) * 449.0
    x[4, ::3] *= 50.0
    xb = x.to(dtype)
    bits = xb.view(torch.int16).numpy().view(np.uint16)
    q, s = oracle.act_split(bits, code)
    assert q.shape == (T * 6, 512) and s.shape == (T * 6,)
    # the scale: smallest power of two with amax / scale <= 448
    xs = xb.float().numpy().astype(np.float64)
    for m in range(6):
        amax = np.abs(xs[m]).max()
        s0 = float(s[T * m])
        if amax == 0:
            assert s0 == 1.0
            continue
        assert np.log2(s0) == np.round(np.log2(s0))
        assert amax / s0 <= 448.0 < amax / (s0 / 2)
        assert all(s[T * m + t] == s0 * 16.0 ** -t for t in range(T))
    rec = _split_recon(q, s, T)
    small = np.abs(xs) < np.repeat(s[::T].astype(np.float64)[:, None], 512, axis=1) * 2.0 ** -6
    assert np.array_equal(rec[~small], xs[~small])
    # below 2^-6 of the scale the subnormal terms keep an absolute error under 2^(E-13)
    assert np.all(np.abs(rec - xs)[small] <= np.repeat(s[::T].astype(np.float64)[:, None], 512, axis=1)[small] * 2.0 ** -13)


def test_w4a16_split_terms_are_rne_of_the_residual(oracle):
    """Each code is torch's RNE e4m3 cast of its residual, the residual recomputed in f32."""
    g = torch.Generator().manual_seed(8)
    x = (torch.randn(3, 256, generator=g) * 5).to(torch.float16)
    q, s = oracle.act_split(x.view(torch.int16).numpy().view(np.uint16), 1)
    for m in range(3):
        r = (x[m].float() / float(s[3 * m])).numpy()
        for t in range(3):
            assert np.array_equal(q[3 * m + t], _torch_e4m3(r))
            r = ((r - torch.from_numpy(q[3 * m + t]).view(torch.float8_e4m3fn).float().numpy()) * 16.0).astype(np.float32)


def test_w4a16_gemm_reference_brute_force(oracle):
    """The W4A16 reference is x @ dequant(W)^T: brute force on a tiny case."""
    N, K, g = 16, 64, 32
    w, sc, z = synth.int4_weight(N, K, g, seed=3, asym=True)
    x = (torch.randn(2, K, generator=torch.Generator().manual_seed(4))).to(torch.bfloat16)
    ref = oracle.w4a16_gemm(x.view(torch.int16).numpy().view(np.uint16), 0, w.numpy(), sc.numpy(), z.numpy(), g)
    codes = ((w.numpy()[:, :, None] >> (4 * np.arange(8))) & 15).reshape(N, K).astype(np.float64)
    zz = ((z.numpy()[:, :, None] >> (4 * np.arange(8))) & 15).reshape(K // g, N).astype(np.float64)
    s64 = sc.numpy().astype(np.float64)
    want = np.zeros((2, N))
    for m in range(2):
        for n in range(N):
            want[m, n] = sum(float(x[m, k]) * (codes[n, k] - zz[k // g, n]) * s64[k // g, n] for k in range(K))
    assert np.allclose(ref, want, rtol=1e-12, atol=1e-12)


def test_nvfp4_dequant_is_two_level(oracle):
    """NVFP4 dequant = e2m1 LUT value * e4m3 block scale (torch's decode) * per-channel global,
    with group 16 (python/minisgl/quant/nvfp4.py:12-18)."""
    N, K = 32, 64
    w, s, glob = synth.nvfp4_weight(N, K, seed=5)
    got = oracle.dequant(w.numpy(), s.view(torch.uint8).numpy(), glob.numpy(), 16, e2m1=True, nvfp4=True)
    codes = ((w.numpy()[:, :, None] >> (4 * np.arange(8))) & 15).reshape(N, K)
    lut = oracle.E2M1_LUT[codes]
    sc = s.to(torch.float32).numpy().astype(np.float64)  # (K/16, N)
    want = lut * sc.T.repeat(16, axis=1) * glob.numpy().astype(np.float64)[:, None]
    assert np.array_equal(got, want)


# ------------------------------------------------------------------------------- W4A16 MoE
def _silu_row(oracle, y1, I, dtype):
    return np.array([oracle.silu_mul(y1[i], y1[I + i], dtype) for i in range(I)], dtype=np.uint16)


@pytest.mark.parametrize("dtype,code", [(torch.float16, 1), (torch.bfloat16, 0)])
def test_w4a16_moe_single_expert_is_the_dense_chain(oracle, dtype, code):
    """One routed expert per token with weight 1: the W4A16 MoE equals the dense chain
    w4a16_gemm -> silu_mul in the dtype -> w4a16_gemm on those values (each piece pinned above),
    with AWQ-style zeros so a dropped zero term would show."""
    T, H, I, E, g = 3, 256, 128, 4, 64
    x = synth.activations(T, H, seed=41, dtype=torch.float32).to(dtype)
    w13, s13, z13 = synth.int4_weight(2 * I, H, g, seed=42, asym=True, E=E)
    w2, s2, z2 = synth.int4_weight(H, I, g, seed=43, asym=True, E=E)
    w13, s13, z13, w2, s2, z2 = (t.numpy() for t in (w13, s13, z13, w2, s2, z2))
    ids = np.array([[2], [0], [2]], dtype=np.int32)
    xb = synth.bits16(x)
    out, h = oracle.w4a16_moe_forward(xb, code, np.ones((T, 1), np.float32), ids, w13, s13, z13, w2, s2, z2)
    for t in range(T):
        e = ids[t, 0]
        y1 = oracle.w4a16_gemm(xb[t:t + 1], code, w13[e], s13[e], z13[e], g)[0]
        hb = _silu_row(oracle, y1, I, code)
        assert np.array_equal(h[t], hb)
        y2 = oracle.w4a16_gemm(hb[None, :], code, w2[e], s2[e], z2[e], g)[0]
        np.testing.assert_allclose(out[t], y2, rtol=1e-12, atol=1e-12)


def test_w4a16_moe_is_linear_in_the_route(oracle):
    """top-k weights (a, b) over experts (e0, e1) give a * out(e0) + b * out(e1), and a dropped
    slot (expert id -1) contributes nothing (MXFP4 weights, fp16 activations)."""
    T, H, I, E = 2, 128, 64, 3
    x = synth.activations(T, H, seed=44, dtype=torch.float32).to(torch.float16)
    w13, s13 = synth.mxfp4_weight(2 * I, H, seed=45, E=E)
    w2, s2 = synth.mxfp4_weight(H, I, seed=46, E=E)
    w13, s13, w2, s2 = w13.numpy(), s13.numpy(), w2.numpy(), s2.numpy()
    xb = synth.bits16(x)
    tw = np.array([[0.625, 0.375], [0.25, 0.75]], dtype=np.float32)
    ids = np.array([[1, 2], [0, 1]], dtype=np.int32)
    both, h = oracle.w4a16_moe_forward(xb, 1, tw, ids, w13, s13, None, w2, s2, None, e2m1=True)
    parts = [oracle.w4a16_moe_forward(xb, 1, np.ones((T, 1), np.float32), ids[:, j:j + 1], w13, s13, None, w2, s2,
                                      None, e2m1=True) for j in range(2)]
    want = tw[:, :1] * parts[0][0] + tw[:, 1:] * parts[1][0]
    np.testing.assert_allclose(both, want, rtol=1e-12, atol=1e-12)
    assert np.array_equal(h[0::2], parts[0][1]) and np.array_equal(h[1::2], parts[1][1])
    dropped = ids.copy()
    dropped[:, 1] = -1
    one, _ = oracle.w4a16_moe_forward(xb, 1, tw, dropped, w13, s13, None, w2, s2, None, e2m1=True)
    np.testing.assert_allclose(one, tw[:, :1] * parts[0][0], rtol=1e-12, atol=1e-12)
