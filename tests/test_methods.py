"""Host-side method layer (CPU): checkpoint buffer declarations, load-time conversion, the
compressed-tensors sign decision, the fused-SwiGLU gate and method selection.

Mirrors python/minisgl/quant/method.py (W4A8LinearMethod, MxFp4LinearMethod,
create_linear_method, _fused_swiglu_ok, ct_packed_sign_convention) and
python/minisgl/layers/moe.py (expert containers, create_moe_quant_method). Pins: shapes from the
reference's declarations; conversions against closed forms (the dequantized value scale * (q - z)
is unchanged by every layout step) and the already-pinned awq/gptq_to_op_layout.
"""
from types import SimpleNamespace

import pytest
import torch

import synth
from conftest import pkg

M_ = pkg("quant.method")
C_ = pkg("quant.config")
K_ = pkg("quant.kernels")
L_ = pkg("layers.moe")

AWQ = C_.QuantConfig(method="awq", bits=4, group_size=128, sym=False)
GPTQ = C_.QuantConfig(method="gptq", bits=4, group_size=128, sym=True)
CT = C_.QuantConfig(method="compressed-tensors", bits=4, group_size=32, sym=True)
CT_ASYM = C_.QuantConfig(method="compressed-tensors", bits=4, group_size=32, sym=False)
MX = C_.QuantConfig(method="compressed-tensors", bits=4, group_size=32, sym=True, weight_type="float",
                    ct_format="mxfp4-pack-quantized")
NV = C_.QuantConfig(method="compressed-tensors", bits=4, group_size=16, sym=True, weight_type="float",
                    ct_format="nvfp4-pack-quantized")
FP8 = C_.QuantConfig(method="compressed-tensors", bits=8, group_size=0, sym=True, weight_type="float")


def _unpack_rows(w: torch.Tensor) -> torch.Tensor:
    """(..., K/8) int32 -> (..., K) codes (nibble j of word i = element 8i+j)."""
    sh = torch.arange(0, 32, 4, dtype=torch.int32)
    return ((w.unsqueeze(-1) >> sh) & 15).reshape(*w.shape[:-1], w.shape[-1] * 8)


def _bell_codes(N, K, seed):
    """Symmetric int4 values q in [-8, 7], peaked at 0 like real quantized weights."""
    g = synth.gen(seed)
    return torch.clamp(torch.round(torch.randn(N, K, generator=g) * 2.0), -8, 7).to(torch.int32)


def _ct_pack(q: torch.Tensor, uint4b8: bool) -> torch.Tensor:
    nib = (q + 8) if uint4b8 else (q & 0xF)
    return synth.pack_rows(nib)


# ---------------------------------------------------------------------------------- declarations
def test_create_weights_checkpoint_shapes():
    N, K = 256, 512
    lay = SimpleNamespace()
    M_.W4A8LinearMethod(GPTQ).create_weights(lay, N, K)
    assert lay.qweight.shape == (K // 8, N) and lay.scales.shape == (K // 128, N) and lay.qzeros.shape == (K // 128, N // 8)
    lay = SimpleNamespace()
    M_.W4A8LinearMethod(AWQ).create_weights(lay, N, K)
    assert lay.qweight.shape == (K, N // 8) and lay.qzeros.shape == (K // 128, N // 8)
    lay = SimpleNamespace()
    M_.W4A8LinearMethod(C_.QuantConfig(method="awq", bits=4, group_size=128, sym=True)).create_weights(lay, N, K)
    assert not hasattr(lay, "qzeros")
    lay = SimpleNamespace()
    M_.W4A8LinearMethod(CT_ASYM).create_weights(lay, N, K)
    assert lay.weight_packed.shape == (N, K // 8) and lay.weight_scale.shape == (N, K // 32)
    assert lay.weight_zero_point.shape == (N // 8, K // 32)
    lay = SimpleNamespace()
    M_.MxFp4LinearMethod(MX).create_weights(lay, N, K)
    assert lay.weight_packed.shape == (N, K // 2) and lay.weight_packed.dtype == torch.uint8
    assert lay.weight_scale.shape == (N, K // 32) and lay.weight_scale.dtype == torch.uint8
    with pytest.raises(AssertionError, match="GPTQ needs"):
        M_.W4A8LinearMethod(GPTQ).create_weights(SimpleNamespace(), 256, 500)


# ---------------------------------------------------------------------------------- conversions
def test_awq_and_gptq_post_load_use_the_layout_converters():
    N, K = 128, 256
    g = synth.gen(3)
    lay = SimpleNamespace(qweight=torch.randint(-2**31, 2**31 - 1, (K, N // 8), generator=g, dtype=torch.int32),
                          scales=torch.rand(K // 128, N, generator=g).to(torch.float16),
                          qzeros=torch.randint(-2**31, 2**31 - 1, (K // 128, N // 8), generator=g, dtype=torch.int32))
    w, s, z = K_.awq_to_op_layout(lay.qweight, lay.scales, lay.qzeros)
    M_.W4A8LinearMethod(AWQ).process_weights_after_load(lay)
    assert torch.equal(lay._w_packed_op, w) and torch.equal(lay._scales_op, s) and torch.equal(lay._zeros_op, z)
    assert not hasattr(lay, "qweight") and not hasattr(lay, "qzeros")
    # GPTQ symmetric: stored zero 7 (+1 = 8) everywhere -> no zero-point tensor at all
    qw = torch.randint(-2**31, 2**31 - 1, (K // 8, N), generator=g, dtype=torch.int32)
    lay = SimpleNamespace(qweight=qw, scales=torch.rand(K // 128, N, generator=g).to(torch.float16),
                          qzeros=torch.full((K // 128, N // 8), 0x77777777, dtype=torch.int32))
    w, _, z = K_.gptq_to_op_layout(lay.qweight, lay.scales, lay.qzeros)
    assert bool((z.view(torch.uint8) == 0x88).all())
    M_.W4A8LinearMethod(GPTQ).process_weights_after_load(lay)
    assert torch.equal(lay._w_packed_op, w) and lay._zeros_op is None


@pytest.mark.parametrize("uint4b8", [True, False])
def test_ct_post_load_dequant_is_exact(uint4b8):
    """compressed-tensors int4 in either packing -> op layout whose dequant equals scale * q."""
    N, K = 128, 256
    q = _bell_codes(N, K, seed=5)
    sc = (torch.rand(N, K // 32, generator=synth.gen(6)) + 0.5).to(torch.float16)
    lay = SimpleNamespace(weight_packed=_ct_pack(q, uint4b8), weight_scale=sc)
    M_.W4A8LinearMethod(CT).process_weights_after_load(lay)
    assert lay._ct_sign.uint4b8 == uint4b8
    assert lay._zeros_op is None
    codes = _unpack_rows(lay._w_packed_op)
    assert torch.equal(codes - 8, q)
    assert lay._scales_op.shape == (K // 32, N) and torch.equal(lay._scales_op, sc.t())


def test_ct_asymmetric_zero_points_share_the_weight_convention():
    N, K = 64, 128
    g = synth.gen(8)
    q = _bell_codes(N, K, seed=9)
    zq = torch.randint(-8, 8, (K // 32, N), generator=g, dtype=torch.int32)  # zero per (group, channel)
    zp_ckpt = synth.pack_rows(zq & 0xF).t().contiguous()  # checkpoint (N/8, G): packed along N, 2-comp
    lay = SimpleNamespace(weight_packed=_ct_pack(q, False), weight_scale=torch.ones(N, K // 32, dtype=torch.float16),
                          weight_zero_point=zp_ckpt)
    M_.W4A8LinearMethod(CT_ASYM).process_weights_after_load(lay)
    z_codes = _unpack_rows(lay._zeros_op)  # (G, N)
    w_codes = _unpack_rows(lay._w_packed_op)  # (N, K)
    # scale * (W_u - Z_u) == scale * (q - zp) for every element
    zq_full = zq.t().repeat_interleave(32, dim=1)
    assert torch.equal(w_codes - z_codes.t().repeat_interleave(32, dim=1), q - zq_full)


def test_ct_sign_decision_samples_whole_tensor_and_refuses_ambiguity():
    # a tensor past the sample budget is sampled in many blocks spread over all of it; both
    # packings of the same values are told apart, and a flat histogram is refused
    N, K = 2048, 1024
    q = _bell_codes(N, K, seed=11)
    packed = _ct_pack(q, True)
    conv = M_.ct_packed_sign_convention(packed)
    assert conv.uint4b8 and conv.blocks > 1 and conv.sampled_words <= 1 << 16
    assert not M_.ct_packed_sign_convention(_ct_pack(q, False)).uint4b8
    uniform = synth.pack_rows(torch.randint(0, 16, (256, 256), generator=synth.gen(1), dtype=torch.int32))
    with pytest.raises(ValueError, match="cannot decide"):
        M_.ct_packed_sign_convention(uniform, min_margin=0.05)
    with pytest.raises(ValueError, match="empty"):
        M_.ct_packed_sign_convention(torch.empty(0, dtype=torch.int32))


def test_ct_sample_blocks_cover_the_tensor():
    raw = torch.arange(1 << 20, dtype=torch.int64).reshape(-1, 1)
    s, blocks, stride = M_._ct_sign_sample(raw)
    idx = s.reshape(-1)
    assert blocks == 512 and idx.numel() == 1 << 16
    assert int(idx[0]) == 0 and int(idx[-1]) == (1 << 20) - 1
    assert len(set(idx.tolist())) == idx.numel()  # no duplicates


def test_mxfp4_post_load_keeps_codes_and_e8m0_bytes():
    N, K = 64, 128
    g = synth.gen(12)
    codes = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int32)
    wpk = (codes[:, 0::2] | (codes[:, 1::2] << 4)).to(torch.uint8)  # low nibble = even k
    ws = torch.randint(110, 130, (N, K // 32), generator=g, dtype=torch.int32).to(torch.uint8)
    lay = SimpleNamespace(weight_packed=wpk, weight_scale=ws)
    M_.MxFp4LinearMethod(MX).process_weights_after_load(lay)
    assert torch.equal(_unpack_rows(lay._w_packed_op), codes)
    assert torch.equal(lay._scales_op, ws.t())


# ---------------------------------------------------------------------------------- gates
def test_fused_swiglu_gate_matches_kernel_constraints():
    w = torch.zeros(256, 512 // 8, dtype=torch.int32)  # N = 256 = 2 x 128
    x = torch.zeros(4, 512, dtype=torch.bfloat16)
    assert M_._fused_swiglu_ok(x, w, 128)
    assert M_._fused_swiglu_ok(x, w, 32) and M_._fused_swiglu_ok(x, w, 64)
    assert not M_._fused_swiglu_ok(torch.zeros(17, 512, dtype=torch.bfloat16), w, 128)  # prefill
    assert not M_._fused_swiglu_ok(x, w, 16)  # 16-wide groups are e2m1-only
    assert M_._fused_swiglu_ok(x, w, 16, weight_is_e2m1=True)  # NVFP4's block
    assert not M_._fused_swiglu_ok(x, torch.zeros(48, 64, dtype=torch.int32), 128)  # inter 24: not whole strips
    assert not M_._fused_swiglu_ok(torch.zeros(4, 500, dtype=torch.bfloat16), torch.zeros(256, 62, dtype=torch.int32), 128)
    tiles = torch.zeros(256 // 16, 4, 1024, dtype=torch.uint8)  # W4 tiles of the same weight
    assert M_._fused_swiglu_ok(x, tiles, 128)


def test_create_linear_method_routes_by_declared_scheme():
    assert isinstance(M_.create_linear_method(AWQ), M_.W4A8LinearMethod)
    assert isinstance(M_.create_linear_method(GPTQ), M_.W4A8LinearMethod)
    assert isinstance(M_.create_linear_method(CT), M_.W4A8LinearMethod)
    assert isinstance(M_.create_linear_method(MX), M_.MxFp4LinearMethod)
    assert isinstance(M_.create_linear_method(None), M_.UnquantizedLinearMethod)
    assert isinstance(M_.create_linear_method(AWQ, quantized=False), M_.UnquantizedLinearMethod)
    assert isinstance(M_.create_linear_method(NV), M_.NvFp4LinearMethod)
    with pytest.raises(NotImplementedError, match="fp8"):
        M_.create_linear_method(FP8)
    assert M_.W4A8LinearMethod(AWQ).supports_producer_actquant


# ---------------------------------------------------------------------------------- MoE
def test_moe_method_selection_and_containers():
    m = L_.create_moe_quant_method(GPTQ)
    assert isinstance(m, L_._W4A8MoEMethod) and m.supports_ep
    assert isinstance(L_.create_moe_quant_method(AWQ).create_experts(4, 64, 256), L_._GroupedAWQExperts)
    assert isinstance(L_.create_moe_quant_method(CT).create_experts(4, 64, 256), L_._GroupedCompressedTensorsExperts)
    mx = L_.create_moe_quant_method(MX)
    assert isinstance(mx, L_._MxFp4MoEMethod)
    assert isinstance(L_.create_moe_quant_method(NV), L_._NvFp4MoEMethod)
    assert isinstance(L_.create_moe_quant_method(NV).create_experts(4, 64, 256), L_._GroupedNvFp4Experts)
    for q in (None, FP8):
        with pytest.raises(NotImplementedError):
            L_.create_moe_quant_method(q)
    # silu and gelu (HF gelu_pytorch_tanh) are served; anything else is refused by name, and the
    # silu-only W4A16 arm refuses gelu (python/minisgl/layers/moe.py:583-593, 678-690)
    L_._check_activation("W4A8", "gelu")
    with pytest.raises(NotImplementedError, match="activation"):
        L_._check_activation("W4A8", "gelu_erf")
    with pytest.raises(NotImplementedError, match="silu-only"):
        L_._reject_w4a16_activation("gelu")
    L_._reject_w4a16_activation("silu")


def test_moe_containers_post_load_per_expert():
    E, N, K = 3, 64, 256
    g = synth.gen(21)
    c = L_.create_moe_quant_method(GPTQ).create_experts(E, N, K)
    assert c.qweight.shape == (E, K // 8, N) and c.scales.shape == (E, K // 128, N)
    c.qweight = torch.randint(-2**31, 2**31 - 1, c.qweight.shape, generator=g, dtype=torch.int32)
    c.scales = torch.rand(c.scales.shape, generator=g).to(torch.float16)
    c.qzeros = torch.full(c.qzeros.shape, 0x77777777, dtype=torch.int32)
    ref = [K_.gptq_to_op_layout(c.qweight[e], c.scales[e], c.qzeros[e]) for e in range(E)]
    c.post_load()
    assert c._w_op.shape == (E, N, K // 8) and c._zeros_op is None
    for e in range(E):
        assert torch.equal(c._w_op[e], ref[e][0]) and torch.equal(c._scales_op[e], ref[e][1])
    assert L_._W4A8MoEMethod.plane(c)[0] is c._w_op
    mx = L_.create_moe_quant_method(MX).create_experts(E, N, K)
    assert mx.weight_packed.shape == (E, N, K // 2) and mx.weight_scale.shape == (E, N, K // 32)
    mx.post_load()
    assert mx._w_op.shape == (E, N, K // 8) and mx._scales_op.shape == (E, K // 32, N)


# ---------------------------------------------------------------------------------- NVFP4 loaders
NV4 = pkg("quant.nvfp4")


def test_nvfp4_global_direction_by_field():
    """compressed-tensors' weight_global_scale divides, modelopt's weight_scale_2 multiplies
    (python/minisgl/quant/nvfp4.py:70-93); an unknown field or a non-positive global is refused."""
    g = torch.tensor(2688.0)
    assert float(NV4.nvfp4_global_multiplier(g, global_field="weight_global_scale")) == float(1.0 / g)
    assert float(NV4.nvfp4_global_multiplier(torch.tensor(2.078e-4), global_field="weight_scale_2")) == \
        float(torch.tensor(2.078e-4))
    with pytest.raises(ValueError, match="unknown"):
        NV4.nvfp4_global_multiplier(g, global_field="global")
    with pytest.raises(ValueError):
        NV4.nvfp4_global_multiplier(torch.tensor(0.0), global_field="weight_scale_2")


def test_nvfp4_split_is_byte_verbatim():
    """The block scale passes through byte for byte (uint8 checkpoints are bitcast, not converted);
    the global becomes an (N,) f32 multiplier vector."""
    raw = torch.arange(0, 126, dtype=torch.uint8)[:120].reshape(8, 15)[:, :12].contiguous()
    block, glob = NV4.split_nvfp4_scale(raw.reshape(8, 12), torch.tensor(4.0), global_field="weight_global_scale")
    assert block.dtype == torch.float8_e4m3fn and torch.equal(block.view(torch.uint8), raw.reshape(8, 12))
    assert glob.shape == (8,) and torch.all(glob == 0.25)
    with pytest.raises(ValueError):
        NV4.split_nvfp4_scale(raw.reshape(8, 12).to(torch.float16), torch.tensor(4.0), global_field="weight_scale_2")


def test_nvfp4_post_load_layouts():
    """Dense and grouped NVFP4 post-load: codes verbatim in the op layout, e4m3 scales group-major,
    the global's f32 bits viewed as int32, and dequant_reference = lut * block * global."""
    N, K = 64, 128
    g = synth.gen(21)
    codes = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int32)
    wpk = (codes[:, 0::2] | (codes[:, 1::2] << 4)).to(torch.uint8)
    ws = (torch.rand(N, K // 16, generator=g) * 6 + 0.25).to(torch.float8_e4m3fn)
    glob = torch.rand(N, generator=g) * 1e-3 + 1e-4
    lay = SimpleNamespace(weight_packed=wpk, weight_scale=ws, weight_global=glob)
    M_.NvFp4LinearMethod(NV).process_weights_after_load(lay)
    assert torch.equal(_unpack_rows(lay._w_packed_op), codes)
    assert torch.equal(lay._scales_op.view(torch.uint8), ws.t().contiguous().view(torch.uint8))
    assert torch.equal(lay._global_op.view(torch.float32), glob)
    deq = NV4.dequant_reference(wpk, ws, glob)
    lut = torch.tensor(pkg("quant.mxfp4").FP4_E2M1_LUT)
    want = lut[codes.long()] * ws.float().repeat_interleave(16, dim=1) * glob[:, None]
    assert torch.equal(deq, want)
    ex = L_.create_moe_quant_method(NV).create_experts(2, N, K)
    ex.weight_packed.copy_(torch.stack([wpk, wpk]))
    ex.weight_scale.copy_(torch.stack([ws, ws]))
    ex.weight_global.copy_(torch.stack([glob, glob * 2]))
    ex.post_load()
    assert ex._scales_op.shape == (2, K // 16, N) and ex._zeros_op.dtype == torch.int32
    assert torch.equal(ex._zeros_op[1].view(torch.float32), glob * 2)
