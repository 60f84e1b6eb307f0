"""GPU: the method layer end to end -- checkpoint-layout buffers, post_load on the device (W4 tiles
made once), apply / apply_swiglu / MoE apply -- against the operator API called on the op layout
(bit-identical, both run the same kernels on the same tiles) and against the CPU oracle.
"""
from types import SimpleNamespace

import pytest
import torch

import synth
from conftest import pkg
from test_gpu_dense import assert_close_to_oracle

pytestmark = pytest.mark.gpu

M_ = pkg("quant.method")
C_ = pkg("quant.config")
L_ = pkg("layers.moe")

AWQ = C_.QuantConfig(method="awq", bits=4, group_size=128, sym=False)
GPTQ = C_.QuantConfig(method="gptq", bits=4, group_size=128, sym=True)
MX = C_.QuantConfig(method="compressed-tensors", bits=4, group_size=32, sym=True, weight_type="float",
                    ct_format="mxfp4-pack-quantized")


def _rand_i32(shape, g):
    return torch.randint(-2**31, 2**31 - 1, shape, generator=g, dtype=torch.int32)


def _awq_layer(N, K, seed, dev):
    g = synth.gen(seed)
    m = M_.W4A8LinearMethod(AWQ)
    lay = SimpleNamespace()
    m.create_weights(lay, N, K)
    lay.qweight = _rand_i32(lay.qweight.shape, g)
    lay.scales = (torch.rand(lay.scales.shape, generator=g) * 0.02 + 1e-3).to(torch.float16)
    lay.qzeros = _rand_i32(lay.qzeros.shape, g)
    ckpt = (lay.qweight.clone(), lay.scales.clone(), lay.qzeros.clone())
    for a in ("qweight", "scales", "qzeros"):
        setattr(lay, a, getattr(lay, a).to(dev))
    m.process_weights_after_load(lay)
    return m, lay, ckpt


@pytest.mark.parametrize("M", [1, 4, 16, 40])
def test_awq_linear_method_matches_operator_and_oracle(kernels, oracle, dev, M):
    N, K = 512, 1024
    m, lay, (qw, sc, qz) = _awq_layer(N, K, seed=31, dev=dev)
    assert lay._w_packed_op.dtype == torch.uint8  # W4 tiles, made once at load
    w_op, s_op, z_op = kernels.awq_to_op_layout(qw, sc, qz)
    x = synth.activations(M, K, seed=M).to(dev)
    bias = torch.randn(N, generator=synth.gen(2)).to(torch.bfloat16).to(dev)
    out = m.apply(lay, x, None)
    out_b = m.apply(lay, x, bias)
    ref_op = kernels.w4a8_linear(x, w_op.to(dev), s_op.to(dev), z_op.to(dev), 128)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_op) and torch.equal(out_b, ref_op + bias)
    xq, xs = oracle.act_quant(synth.bits16(x.cpu()), 0)
    ref = oracle.gemm(xq, xs, w_op.numpy(), s_op.numpy(), z_op.numpy(), 128, False)
    assert_close_to_oracle(out, ref, f"AWQ method M={M}")


def test_awq_apply_swiglu_fires_at_decode_and_is_bit_exact(kernels, dev):
    N, K = 512, 1024  # merged gate_up, inter 256
    m, lay, _ = _awq_layer(N, K, seed=41, dev=dev)
    x = synth.activations(4, K, seed=3).to(dev)
    fused = m.apply_swiglu(lay, x)
    y = m.apply(lay, x, None)
    gh, uh = y[:, : N // 2], y[:, N // 2:]
    ref = (gh.float() / (1.0 + torch.exp(-gh.float()))).to(x.dtype) * uh
    torch.cuda.synchronize()
    assert fused is not None and torch.equal(fused, ref)
    assert m.apply_swiglu(lay, synth.activations(17, K, seed=4).to(dev)) is None  # prefill: caller unfuses


def test_gptq_symmetric_method_drops_zeros_and_matches_oracle(kernels, oracle, dev):
    N, K = 256, 2048
    g = synth.gen(51)
    m = M_.W4A8LinearMethod(GPTQ)
    lay = SimpleNamespace()
    m.create_weights(lay, N, K)
    qw = _rand_i32(lay.qweight.shape, g)
    sc = (torch.rand(lay.scales.shape, generator=g) * 0.02 + 1e-3).to(torch.float16)
    lay.qweight, lay.scales = qw.to(dev), sc.to(dev)
    lay.qzeros = torch.full(lay.qzeros.shape, 0x77777777, dtype=torch.int32, device=dev)
    m.process_weights_after_load(lay)
    assert lay._zeros_op is None
    w_op, s_op, _ = kernels.gptq_to_op_layout(qw, sc, torch.full((K // 128, N // 8), 0x77777777, dtype=torch.int32))
    x = synth.activations(2, K, seed=5).to(dev)
    out = m.apply(lay, x, None)
    torch.cuda.synchronize()
    xq, xs = oracle.act_quant(synth.bits16(x.cpu()), 0)
    assert_close_to_oracle(out, oracle.gemm(xq, xs, w_op.numpy(), s_op.numpy(), None, 128, False), "GPTQ sym method")


def test_mxfp4_linear_method(kernels, oracle, dev):
    N, K = 256, 1024
    g = synth.gen(61)
    codes = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int32)
    wpk = (codes[:, 0::2] | (codes[:, 1::2] << 4)).to(torch.uint8)
    ws = torch.randint(119, 128, (N, K // 32), generator=g, dtype=torch.int32).to(torch.uint8)
    m = M_.create_linear_method(MX)
    lay = SimpleNamespace(weight_packed=wpk.to(dev), weight_scale=ws.to(dev))
    m.process_weights_after_load(lay)
    x = synth.activations(3, K, seed=6).to(dev)
    out = m.apply(lay, x, None)
    torch.cuda.synchronize()
    xq, xs = oracle.act_quant(synth.bits16(x.cpu()), 0)
    ref = oracle.gemm(xq, xs, synth.pack_rows(codes).numpy(), ws.t().contiguous().numpy(), None, 32, True)
    assert_close_to_oracle(out, ref, "MXFP4 method")


def _gptq_experts(kernels, dev, E, H, I):
    """A GPTQ MoE method and expert pair after post_load, and the op-layout (w, scales) of each."""
    g = synth.gen(71)
    m = L_.create_moe_quant_method(GPTQ)
    w13, w2 = m.create_experts(E, 2 * I, H), m.create_experts(E, H, I)
    for c in (w13, w2):
        c.qweight = _rand_i32(c.qweight.shape, g)
        c.scales = (torch.rand(c.scales.shape, generator=g) * 0.02 + 1e-3).to(torch.float16)
        c.qzeros = torch.full(c.qzeros.shape, 0x77777777, dtype=torch.int32)
    ops = []
    for c in (w13, w2):
        parts = [kernels.gptq_to_op_layout(c.qweight[e], c.scales[e], c.qzeros[e]) for e in range(E)]
        ops.append((torch.stack([p[0] for p in parts]).to(dev), torch.stack([p[1] for p in parts]).to(dev)))
        c.qweight, c.scales, c.qzeros = c.qweight.to(dev), c.scales.to(dev), c.qzeros.to(dev)
        c.post_load()
    return m, w13, w2, ops


def test_moe_method_matches_operator(kernels, dev):
    """GPTQ experts through the MoE method == w4a8_moe on the op layout (same route, same tiles)."""
    E, H, I, T, k = 8, 256, 128, 5, 2
    m, w13, w2, ops = _gptq_experts(kernels, dev, E, H, I)
    assert w13._zeros_op is None and w13._w_op.dtype == torch.uint8
    x = synth.activations(T, H, seed=8).to(dev)
    logits = synth.router_logits(T, E, seed=9).to(dev)
    out = m.apply(w13, w2, x, router_logits=logits, topk_weights=None, topk_ids=None, top_k=k, renormalize=True,
                  activation="silu", apply_router_weight_on_input=False)
    ref = kernels.w4a8_moe(x, ops[0][0], ops[0][1], None, ops[1][0], ops[1][1], None, logits, k, True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    # the EP shard kernel with a precomputed route is the same computation
    tw, ti = kernels._moe_route(logits, k, True, E)
    out_ep = m.ep_local(w13, w2, x, tw, ti, top_k=k, renormalize=True)
    torch.cuda.synchronize()
    assert torch.equal(out_ep, out)


NV = C_.QuantConfig(method="compressed-tensors", bits=4, group_size=16, sym=True, weight_type="float",
                    ct_format="nvfp4-pack-quantized")


def _nv_layer(N, K, seed, dev):
    g = synth.gen(seed)
    codes = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int32)
    m = M_.create_linear_method(NV)
    lay = SimpleNamespace()
    m.create_weights(lay, N, K)
    lay.weight_packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).to(torch.uint8).to(dev)
    ws = (torch.rand(N, K // 16, generator=g) * 6 + 0.25).to(torch.float8_e4m3fn)
    glob = torch.rand(N, generator=g) * 1e-3 + 1e-4
    lay.weight_scale, lay.weight_global = ws.to(dev), glob.to(dev)
    m.process_weights_after_load(lay)
    return m, lay, codes, ws, glob


def test_nvfp4_linear_method(kernels, oracle, dev):
    """NVFP4 checkpoint buffers -> post_load -> apply, against the oracle's two-level dequant."""
    N, K = 256, 1024
    m, lay, codes, ws, glob = _nv_layer(N, K, 81, dev)
    for M in (1, 3, 40):
        x = synth.activations(M, K, seed=M).to(dev)
        out = m.apply(lay, x, None)
        torch.cuda.synchronize()
        xq, xs = oracle.act_quant(synth.bits16(x.cpu()), 0)
        ref = oracle.gemm(xq, xs, synth.pack_rows(codes).numpy(), ws.t().contiguous().view(torch.uint8).numpy(),
                          glob.numpy(), 16, e2m1=True, nvfp4=True)
        assert_close_to_oracle(out, ref, f"NVFP4 method M={M}")


def test_w4a16_opt_in_routes_methods(kernels, dev, monkeypatch):
    """MINISGL_MOE_W4A16 != "0": the dense methods run the W4A16 arm (no producer pair advertised),
    bit-identical to w4a16_linear on the same tiles; the int4 MoE method runs w4a16_moe (apply and
    ep_local), bit-identical to the operator on the op layout."""
    eng = pkg("_hip_engage")
    N, K = 256, 512
    m, lay, *_ = _nv_layer(N, K, 83, dev)
    x = synth.activations(4, K, seed=4).to(dev)
    monkeypatch.setattr(kernels, "MOE_W4A16", "1")
    assert not m.supports_producer_actquant
    before = eng.counts()
    out = m.apply(lay, x, None)
    ref = kernels.w4a16_linear(x, lay._w_packed_op, lay._scales_op, lay._global_op, 16, N, weight_is_e2m1=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert eng.counts_delta(before).get("w4a8_mi355x.w4a16_gemv+e2m1", 0) >= 1
    E, H, I, k = 8, 256, 128, 2
    mm, w13, w2, ops = _gptq_experts(kernels, dev, E, H, I)
    xm = synth.activations(5, H, seed=10).to(dev)
    logits = synth.router_logits(5, E, seed=11).to(dev)
    before = eng.counts()
    out = mm.apply(w13, w2, xm, router_logits=logits, topk_weights=None, topk_ids=None, top_k=k, renormalize=True,
                   activation="silu", apply_router_weight_on_input=False)
    ref = kernels.w4a16_moe(xm, ops[0][0], ops[0][1], None, ops[1][0], ops[1][1], None, H, I, 128,
                            router_logits=logits, top_k=k, renormalize=True)
    tw, ti = kernels._moe_route(logits, k, True, E)
    out_ep = mm.ep_local(w13, w2, xm, tw, ti, top_k=k, renormalize=True)
    torch.cuda.synchronize()
    assert out.dtype == xm.dtype and torch.equal(out, ref) and torch.equal(out_ep, out)
    assert eng.counts_delta(before).get("w4a8_mi355x.w4a16_moe_silu_split", 0) >= 3


def test_nvfp4_moe_method_matches_operator(kernels, dev, monkeypatch):
    E, H, I, T, k = 8, 256, 128, 5, 2
    g = synth.gen(91)
    m = L_.create_moe_quant_method(NV)
    w13, w2 = m.create_experts(E, 2 * I, H), m.create_experts(E, H, I)
    ops = []
    for c, (n, kk) in ((w13, (2 * I, H)), (w2, (H, I))):
        codes = torch.randint(0, 16, (E, n, kk), generator=g, dtype=torch.int32)
        c.weight_packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).to(torch.uint8).to(dev)
        c.weight_scale = (torch.rand(E, n, kk // 16, generator=g) * 6 + 0.25).to(torch.float8_e4m3fn).to(dev)
        c.weight_global = (torch.rand(E, n, generator=g) * 1e-2 + 1e-3).to(dev)
        ops.append((synth.pack_rows(codes).to(dev), c.weight_scale.transpose(1, 2).contiguous(),
                    c.weight_global.view(torch.int32).clone()))
        c.post_load()
    x = synth.activations(T, H, seed=8).to(dev)
    logits = synth.router_logits(T, E, seed=9).to(dev)
    out = m.apply(w13, w2, x, router_logits=logits, topk_weights=None, topk_ids=None, top_k=k, renormalize=True,
                  activation="silu", apply_router_weight_on_input=False)
    ref = kernels.w4a8_moe(x, ops[0][0], ops[0][1], ops[0][2], ops[1][0], ops[1][1], ops[1][2], logits, k, True,
                           weight_is_e2m1=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    # W4A16 opt-in: forwards of up to 2 tokens run w4a16_moe_decode, wider ones stay W4A8
    monkeypatch.setattr(kernels, "MOE_W4A16", "1")
    for rows in (1, 2, T):
        xs, ls = x[:rows], logits[:rows]
        got = m.apply(w13, w2, xs, router_logits=ls, topk_weights=None, topk_ids=None, top_k=k, renormalize=True,
                      activation="silu", apply_router_weight_on_input=False)
        if rows <= 2:
            want = kernels.w4a16_moe_decode(xs, *ops[0], *ops[1], H, router_logits=ls, top_k=k, renormalize=True)
        else:
            want = kernels.w4a8_moe(xs, *ops[0], *ops[1], ls, k, True, weight_is_e2m1=True)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"rows={rows}"


def test_loader_builds_serving_layers(kernels, dev, tmp_path):
    """Checkpoint tensors -> quant.loader -> method.apply on the GPU, bit-identical to the operator
    called on the same tensors converted by hand (AWQ gate_up from two parts, NVFP4 modelopt leaf)."""
    from safetensors.torch import save_file
    LD = pkg("quant.loader")
    K, I, g = 512, 128, 128
    gen = synth.gen(95)
    t = {}
    for p in ("gate_proj", "up_proj"):
        t[f"m.{p}.qweight"] = _rand_i32((K, I // 8), gen)
        t[f"m.{p}.scales"] = (torch.rand(K // g, I, generator=gen) * 0.02 + 1e-3).to(torch.float16)
        t[f"m.{p}.qzeros"] = _rand_i32((K // g, I // 8), gen)
    codes = torch.randint(0, 256, (I, K // 2), generator=gen, dtype=torch.int32).to(torch.uint8)
    t["n.weight"] = codes
    t["n.weight_scale"] = (torch.rand(I, K // 16, generator=gen) * 4 + 0.5).to(torch.float8_e4m3fn)
    t["n.weight_scale_2"] = torch.tensor(2e-3)
    save_file(t, str(tmp_path / "c.safetensors"))
    tensors = LD.read_safetensors([tmp_path / "c.safetensors"])
    m, lay = LD.build_linear(AWQ, "m.gate_up_proj", K, 2 * I, tensors, parts=["m.gate_proj", "m.up_proj"], device=dev)
    x = synth.activations(3, K, seed=1).to(dev)
    ops = [kernels.awq_to_op_layout(t[f"m.{p}.qweight"], t[f"m.{p}.scales"], t[f"m.{p}.qzeros"]) for p in ("gate_proj", "up_proj")]
    w = torch.cat([o[0] for o in ops], 0).to(dev)
    s = torch.cat([o[1] for o in ops], 1).to(dev)
    z = torch.cat([o[2] for o in ops], 1).to(dev)
    assert torch.equal(m.apply(lay, x, None), kernels.w4a8_linear(x, w, s, z, g))
    assert torch.equal(m.apply_swiglu(lay, x), kernels.w4a8_linear_silu(x, w, s, z, g))
    NV_ = C_.QuantConfig.from_hf({"quantization_config": {"quant_method": "modelopt", "quant_algo": "NVFP4"}})
    mn, ln = LD.build_linear(NV_, "n", K, I, tensors, device=dev)
    nv4 = pkg("quant.nvfp4")
    conv = nv4.convert_nvfp4_weight(codes, t["n.weight_scale"])
    glob = torch.full((I,), float(torch.tensor(2e-3)), dtype=torch.float32, device=dev)
    ref = kernels.w4a8_linear(x, conv["w_packed"].to(dev), conv["scales"].t().contiguous().to(dev), glob, 16,
                              weight_is_e2m1=True)
    torch.cuda.synchronize()
    assert torch.equal(mn.apply(ln, x, None), ref)
