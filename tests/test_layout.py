"""Load-time layout conversion: checkpoint -> op layout (reference contract) -> W4 tiles.

The op-layout converters are pinned the way the reference pins them
(tools/qwen3_5_moe_awq_convert_test.py:40-97, tools/qwen2_moe_gptq_convert_test.py:35-50): the
dequantized op layout must equal the dequantized checkpoint exactly. The checkpoint tensors are
built here from known codes, so the checkpoint dequant is itself checked against those codes.
"""
import numpy as np
import pytest
import torch

import synth
from conftest import pkg

AWQ_ORDER = [0, 2, 4, 6, 1, 3, 5, 7]  # nibble j of an AWQ word holds channel 8i + AWQ_ORDER[j]
REV = [0, 4, 1, 5, 2, 6, 3, 7]


def _pack_words(vals: np.ndarray) -> np.ndarray:
    v = vals.astype(np.int64).reshape(*vals.shape[:-1], -1, 8)
    w = (v << (4 * np.arange(8))).sum(-1)
    return (w & 0xFFFFFFFF).astype(np.uint32).view(np.int32)


def _unpack_words(w: np.ndarray) -> np.ndarray:
    u = (w.astype(np.uint32)[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    return u.reshape(*w.shape[:-1], -1).astype(np.int64)


def _awq_checkpoint(K, N, g, seed):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, (K, N))
    zeros = rng.integers(0, 16, (K // g, N))
    scales = (np.abs(rng.standard_normal((K // g, N))) * 0.02 + 1e-4).astype(np.float16)
    qweight = _pack_words(codes.reshape(K, N // 8, 8)[:, :, AWQ_ORDER].reshape(K, N))
    qzeros = _pack_words(zeros.reshape(K // g, N // 8, 8)[:, :, AWQ_ORDER].reshape(K // g, N))
    return codes, zeros, scales, qweight, qzeros


def _awq_ref_dequant(qweight, scales, qzeros, g):
    """tools/qwen3_5_moe_awq_convert_test.py:40-54 restated: (K, N) f32."""
    K, Np = qweight.shape
    N = Np * 8
    q = _unpack_words(qweight).reshape(K, Np, 8)[:, :, REV].reshape(K, N)
    z = _unpack_words(qzeros).reshape(qzeros.shape[0], Np, 8)[:, :, REV].reshape(-1, N)
    gi = np.arange(K) // g
    return scales.astype(np.float64)[gi] * (q - z[gi])


def _op_dequant(w_packed, scales_op, zeros_op, K, g):
    """Op layout dequant with the group-major scales/zeros contract (python/minisgl/quant/
    kernels.py:265-268, 286-291): (N, K) f64."""
    q = _unpack_words(w_packed)
    N = q.shape[0]
    z = _unpack_words(zeros_op) if zeros_op is not None else np.full((K // g, N), 8)
    gi = np.arange(K) // g
    return scales_op.astype(np.float64).T[:, gi] * (q - z.T[:, gi])


def test_awq_to_op_layout_dequant_identical():
    K, N, g = 256, 64, 128
    codes, zeros, scales, qweight, qzeros = _awq_checkpoint(K, N, g, 1)
    ref = _awq_ref_dequant(qweight, scales, qzeros, g)
    # the checkpoint dequant is the known-code dequant
    assert np.array_equal(ref, scales.astype(np.float64)[np.arange(K) // g] * (codes - zeros[np.arange(K) // g]))
    K_ = pkg("quant.kernels")
    w, s, z = K_.awq_to_op_layout(torch.from_numpy(qweight), torch.from_numpy(scales), torch.from_numpy(qzeros))
    assert tuple(w.shape) == (N, K // 8) and tuple(s.shape) == (K // g, N) and tuple(z.shape) == (K // g, N // 8)
    assert s.dtype == torch.float16 and w.dtype == torch.int32 and z.dtype == torch.int32
    got = _op_dequant(w.numpy(), s.numpy(), z.numpy(), K, g)
    assert np.array_equal(got.T, ref)
    # natural nibble order along K
    assert np.array_equal(_unpack_words(w.numpy()), codes.T)


def test_gptq_to_op_layout_dequant_identical():
    K, N, g = 256, 32, 128
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 16, (K, N))
    stored = rng.integers(0, 15, (K // g, N))            # zero point = stored + 1 <= 15
    scales = (np.abs(rng.standard_normal((K // g, N))) * 0.02).astype(np.float16)
    qweight = _pack_words(codes.T).T.copy()               # (K/8, N): word kp nibble j = k 8kp+j
    qweight = np.ascontiguousarray(_pack_words(codes.T.reshape(N, K)).T)
    qzeros = _pack_words(stored)
    # tools/qwen2_moe_gptq_convert_test.py:35-48 restated
    q = _unpack_words(np.ascontiguousarray(qweight.T)).T  # (K, N)
    assert np.array_equal(q, codes)
    gi = np.arange(K) // g
    ref = scales.astype(np.float64)[gi] * (codes - (stored + 1)[gi])
    K_ = pkg("quant.kernels")
    w, s, z = K_.gptq_to_op_layout(torch.from_numpy(qweight), torch.from_numpy(scales), torch.from_numpy(qzeros))
    got = _op_dequant(w.numpy(), s.numpy(), z.numpy(), K, g)
    assert np.array_equal(got.T, ref)


def test_gptq_symmetric_stores_seven():
    K, N, g = 128, 16, 128
    qw = torch.zeros((K // 8, N), dtype=torch.int32)
    qz = torch.from_numpy(_pack_words(np.full((K // g, N), 7)))
    _, _, z = pkg("quant.kernels").gptq_to_op_layout(qw, torch.ones(K // g, N, dtype=torch.float16), qz)
    assert (_unpack_words(z.numpy()) == 8).all()


def test_mxfp4_converters_pass_codes_and_e8m0_through():
    """python/minisgl/quant/mxfp4.py:134-206 contract, tests/mxfp4_e8m0_test.py:45-62 checks."""
    mx = pkg("quant.mxfp4")
    E, N, K = 2, 16, 128
    g = torch.Generator().manual_seed(3)
    packed = torch.randint(0, 256, (E, N, K // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    scale = torch.randint(100, 140, (E, N, K // 32), generator=g, dtype=torch.int32).to(torch.uint8)
    conv = mx.convert_mxfp4_moe_e8m0(packed, scale)
    assert conv["scales"].dtype == torch.uint8 and torch.equal(conv["scales"], scale)
    assert conv["w_zeros"] is None and conv["group_size"] == 32 and conv["scale_is_e8m0"] is True
    # codes verbatim: low nibble = even k
    codes = _unpack_words(conv["w_packed"].numpy())
    p = packed.numpy().astype(np.int64)
    assert np.array_equal(codes[..., 0::2], p & 15) and np.array_equal(codes[..., 1::2], p >> 4)
    one = mx.convert_mxfp4_weight(packed[0], scale[0])
    assert torch.equal(one["w_packed"], conv["w_packed"][0])
    deq = mx.dequant_reference(packed[0], scale[0]).numpy()
    lut = np.array(mx.FP4_E2M1_LUT)
    ref = lut[codes[0]] * 2.0 ** (np.repeat(scale[0].numpy().astype(np.float64), 32, 1) - 127)
    assert np.array_equal(deq, ref)


def test_e8m0_health_report():
    mx = pkg("quant.mxfp4")
    scale = torch.cat([torch.full((30,), 127, dtype=torch.uint8), torch.full((2,), 167, dtype=torch.uint8)]).view(1, 1, 32)
    info = mx.e8m0_scale_health(scale)
    assert info["would_saturate_fp16"] == 2 and info["e8m0_nan_groups"] == 0 and info["exp_max"] == 40


def test_e8m0_health_report_against_brute_force():
    """Every field against a per-code count over all 256 codes (0 = the 2^-127 zero code, 255 = NaN,
    codes outside fp16's normal exponents -14..15 saturate, code 0 excepted)."""
    mx = pkg("quant.mxfp4")
    g = torch.Generator().manual_seed(7)
    for lo, hi in [(0, 256), (100, 140), (120, 130), (0, 2), (250, 256)]:
        scale = torch.randint(lo, hi, (3, 40, 24), generator=g, dtype=torch.int32).to(torch.uint8)
        v = scale.numpy().astype(np.int64).ravel()
        e = v - 127
        info = mx.e8m0_scale_health(scale)
        assert info["exp_min"] == e.min() and info["exp_max"] == e.max()
        assert info["e8m0_nan_groups"] == int((v == 255).sum())
        assert info["e8m0_zero_code_groups"] == int((v == 0).sum())
        assert info["would_saturate_fp16"] == int(((e > 15) | ((e < -14) & (v != 0))).sum())


def test_mxfp4_word_view_is_the_nibble_repack():
    """The converters' word view equals packing the unpacked nibbles explicitly (code j at bits 4j)."""
    mx = pkg("quant.mxfp4")
    g = torch.Generator().manual_seed(9)
    packed = torch.randint(0, 256, (3, 48, 64), generator=g, dtype=torch.int32).to(torch.uint8)
    words = mx.convert_mxfp4_moe_e8m0(packed, torch.full((3, 48, 4), 127, dtype=torch.uint8))["w_packed"]
    for i in range(3):
        assert torch.equal(words[i], mx.pack_codes_to_int32(mx.unpack_e2m1_nibbles(packed[i])))


# ------------------------------------------------------------------------------------ W4 tiles
def tile_reference(w_packed: np.ndarray, K: int, e2m1: bool) -> np.ndarray:
    """numpy restatement of the W4 tile layout: (N/16, KT, 64 lanes, 16 bytes)."""
    codes = _unpack_words(w_packed)  # (N, K)
    N = codes.shape[0]
    KT = (K + 127) // 128
    out = np.zeros((N // 16, KT, 64, 4), dtype=np.uint32)
    for lane in range(64):
        q, c16 = lane >> 4, lane & 15
        n = np.arange(N // 16)[:, None] * 16 + c16  # (NS, 1)
        for kt in range(KT):
            if e2m1:
                for d in range(4):
                    k0 = kt * 128 + 32 * q + 8 * d
                    if k0 < K:
                        out[:, kt, lane, d] = w_packed[n[:, 0], k0 // 8].astype(np.uint32)
            else:
                for e in range(32):
                    k = kt * 128 + (16 * q + e if e < 16 else 64 + 16 * q + e - 16)
                    if k >= K:
                        continue
                    qv = codes[n[:, 0], k]
                    c = np.where(qv >= 8, qv - 8, 15 - qv).astype(np.uint32)
                    d, within = e >> 3, e & 7
                    out[:, kt, lane, d] |= c << (8 * (within & 3) + (4 if within >= 4 else 0))
    return out.view(np.uint8).reshape(N // 16, KT, 1024)


def test_tile_codes_decode_to_q_minus_7_5():
    """The sign-magnitude tile code c = q>=8 ? q-8 : 15-q decodes to q - 7.5 for every q."""
    for q in range(16):
        c = q - 8 if q >= 8 else 15 - q
        v = (-1 if c & 8 else 1) * ((c & 7) + 0.5)
        assert v == q - 7.5


def test_unpack_lut_bytes_are_e4m3_of_half_steps(oracle):
    lut = [0x30, 0x3C, 0x42, 0x46, 0x49, 0x4B, 0x4D, 0x4F]
    assert oracle.e4m3_decode(np.array(lut)).tolist() == [t + 0.5 for t in range(8)]
    assert oracle.e4m3_decode(np.array([0xB0]))[0] == -0.5 and oracle.e4m3_decode(np.array([0x30]))[0] == 0.5
