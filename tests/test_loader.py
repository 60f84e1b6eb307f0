"""Checkpoint ingestion on the CPU: QuantConfig.from_hf header detection and the safetensors loader
(quant/loader.py) filling the methods' declared buffers, fused projections and stacked experts.

Each case builds a small synthetic checkpoint in the producer's own tensor names and dtypes, writes
it with safetensors, reads it back through the loader and compares the converted layouts with the
operator-level conversions of the same tensors.
"""
import pytest
import torch
from safetensors.torch import save_file

import synth
from conftest import pkg

C_ = pkg("quant.config")
K_ = pkg("quant.kernels")
LD = pkg("quant.loader")
M_ = pkg("quant.method")
Q = C_.QuantConfig


# ------------------------------------------------------------------------------------ from_hf
def test_from_hf_awq_gptq():
    q = Q.from_hf({"quantization_config": {"quant_method": "awq", "bits": 4, "group_size": 128, "zero_point": True,
                                           "modules_to_not_convert": ["lm_head", "model.language_model.layers.0.mlp.gate"]}})
    assert q.is_awq and not q.sym and q.group_size == 128 and q.is_int4
    assert q.ignore == ("lm_head", "model.layers.0.mlp.gate")  # multimodal infix stripped
    assert q.for_module("lm_head") is None and q.for_module("model.layers.1.mlp.up_proj") is q
    g = Q.from_hf({"text_config": {"quantization_config": {"quant_method": "gptq", "bits": 4, "group_size": 32,
                                                           "sym": False, "desc_act": True}}})
    assert g.is_gptq and not g.sym and g.desc_act and g.group_size == 32
    assert Q.from_hf({"quantization_config": {"quant_method": "bitsandbytes"}}) is None
    assert Q.from_hf({}) is None


def test_from_hf_compressed_tensors_formats():
    def ct(weights, fmt, **extra):
        return {"quantization_config": {"quant_method": "compressed-tensors", "format": fmt,
                                        "config_groups": {"group_0": {"targets": ["Linear"], "weights": weights}},
                                        **extra}}
    i4 = Q.from_hf(ct({"num_bits": 4, "type": "int", "symmetric": False, "group_size": 32}, "pack-quantized"))
    assert i4.is_compressed_tensors and i4.is_int4 and not i4.sym and i4.group_size == 32
    mx = Q.from_hf(ct({"num_bits": 4, "type": "float", "group_size": 32}, "mxfp4-pack-quantized"))
    assert mx.weight_is_e2m1 and not mx.is_nvfp4
    nv = Q.from_hf(ct({"num_bits": 4, "type": "float", "group_size": 16}, "nvfp4-pack-quantized", ignore=["lm_head"]))
    assert nv.is_nvfp4 and not nv.weight_is_e2m1 and nv.group_size == 16 and nv.for_module("lm_head") is None
    assert isinstance(M_.create_linear_method(nv), M_.NvFp4LinearMethod)


def test_from_hf_modelopt_nvfp4_and_globs():
    q = Q.from_hf({"quantization_config": {"quant_method": "modelopt", "quant_algo": "NVFP4",
                                           "ignore": ["lm_head", "model.layers.*.mlp.gate", "mtp.*"]}})
    assert q.is_nvfp4 and q.group_size == 16 and q.bits == 4
    assert q.for_module("model.layers.3.mlp.gate") is None  # glob -> anchored regex
    assert q.for_module("model.layers.3.mlp.gate_proj") is q
    assert q.for_module("mtp.fc") is None and q.for_module("model.mtp_proj") is q
    assert Q.from_hf({"quantization_config": {"quant_method": "modelopt", "quant_algo": "W4A16_SOMETHING"}}) is None


def test_from_hf_mixed_precision_first_match_catchall_last():
    """A class-name catch-all declared first must not shadow the explicit fp8 targets (config.py:583-599)."""
    q = Q.from_hf({"quantization_config": {
        "quant_method": "compressed-tensors", "format": "mixed-precision", "ignore": ["lm_head"],
        "config_groups": {
            "group_0": {"targets": ["Linear"], "format": "nvfp4-pack-quantized",
                        "weights": {"num_bits": 4, "type": "float", "group_size": 16}},
            "group_1": {"targets": ["re:.*self_attn\\.(q|k|v|o)_proj$"],
                        "weights": {"num_bits": 8, "type": "float", "strategy": "channel"},
                        "input_activations": {"num_bits": 8, "type": "float"}}}}})
    assert q.for_module("model.layers.0.self_attn.q_proj").is_fp8_w8a8
    assert q.for_module("model.layers.0.self_attn.q_proj").act_type == "fp8"
    assert q.for_module("model.layers.0.mlp.down_proj").is_nvfp4
    assert q.for_module("lm_head") is None


# ------------------------------------------------------------------------------------ loader
def _roundtrip(tmp_path, tensors):
    path = tmp_path / "ckpt.safetensors"
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(path))
    return LD.read_safetensors([path])


def _rand_i32(shape, g):
    return torch.randint(-2**31, 2**31 - 1, shape, generator=g, dtype=torch.int32)


def test_awq_gate_up_fused_from_parts(tmp_path):
    """gate_proj + up_proj AWQ tensors -> one gate_up layer whose op layout is the per-part op
    layouts concatenated along N (bf16 scales in the file are value-converted to fp16)."""
    K, I, g = 256, 64, 128
    q = Q(method="awq", bits=4, group_size=g, sym=False)
    gen = synth.gen(3)
    t = {}
    for p in ("gate_proj", "up_proj"):
        t[f"m.{p}.qweight"] = _rand_i32((K, I // 8), gen)
        t[f"m.{p}.scales"] = (torch.rand(K // g, I, generator=gen) * 0.02).to(torch.bfloat16)
        t[f"m.{p}.qzeros"] = _rand_i32((K // g, I // 8), gen)
    tensors = _roundtrip(tmp_path, t)
    m, lay = LD.build_linear(q, "m.gate_up_proj", K, 2 * I, tensors, parts=["m.gate_proj", "m.up_proj"], device="cpu")
    assert isinstance(m, M_.W4A8LinearMethod)
    ops = [K_.awq_to_op_layout(t[f"m.{p}.qweight"], t[f"m.{p}.scales"].to(torch.float16), t[f"m.{p}.qzeros"])
           for p in ("gate_proj", "up_proj")]
    assert torch.equal(lay._w_packed_op, torch.cat([o[0] for o in ops], dim=0))
    assert torch.equal(lay._scales_op, torch.cat([o[1] for o in ops], dim=1))
    assert torch.equal(lay._zeros_op, torch.cat([o[2] for o in ops], dim=1))


def test_loader_refusals(tmp_path):
    K, N, g = 256, 64, 128
    q = Q(method="gptq", bits=4, group_size=g, sym=True)
    gen = synth.gen(4)
    good = {"m.qweight": _rand_i32((K // 8, N), gen), "m.scales": torch.rand(K // g, N).to(torch.float16),
            "m.qzeros": torch.full((K // g, N // 8), 0x77777777, dtype=torch.int32)}
    with pytest.raises(TypeError, match="dtype mismatch"):
        LD.build_linear(q, "m", K, N, dict(good, **{"m.qweight": good["m.qweight"].to(torch.int64)}), device="cpu")
    with pytest.raises(ValueError, match="shape"):
        LD.build_linear(q, "m", K, N, dict(good, **{"m.scales": good["m.scales"][:1]}), device="cpu")
    with pytest.raises(KeyError, match="m.qzeros"):
        LD.build_linear(q, "m", K, N, {k: v for k, v in good.items() if k != "m.qzeros"}, device="cpu")
    m, lay = LD.build_linear(q, "m", K, N, good, device="cpu")
    assert lay._zeros_op is None  # GPTQ's stored all-8 zeros collapse to the symmetric path


def test_ignored_module_loads_unquantized(tmp_path):
    q = Q(method="awq", bits=4, group_size=128, sym=False, ignore=("lm_head",))
    w = torch.randn(64, 32).to(torch.bfloat16)
    m, lay = LD.build_linear(q, "lm_head", 32, 64, {"lm_head.weight": w}, device="cpu")
    assert isinstance(m, M_.UnquantizedLinearMethod) and lay.weight.dtype == torch.bfloat16
    assert torch.equal(lay.weight, w)


@pytest.mark.parametrize("producer", ["compressed-tensors", "modelopt"])
def test_nvfp4_leaf_global_direction(tmp_path, producer):
    """NVFP4 leaves: compressed-tensors' weight_global_scale is a divisor, modelopt's weight_scale_2 a
    multiplier; both end as the same per-channel multiplier vector. uint8 block-scale bytes are
    bitcast; modelopt's packed codes are named `weight`."""
    K, I = 128, 32
    q = Q(method="compressed-tensors", bits=4, group_size=16, sym=True, weight_type="float",
          ct_format="nvfp4-pack-quantized")
    gen = synth.gen(5)
    t = {}
    for j, p in enumerate(("gate_proj", "up_proj")):
        codes = torch.randint(0, 256, (I, K // 2), generator=gen, dtype=torch.int32).to(torch.uint8)
        sc = (torch.rand(I, K // 16, generator=gen) * 4 + 0.5).to(torch.float8_e4m3fn)
        mul = 0.001 * (j + 1)
        if producer == "compressed-tensors":
            t[f"m.{p}.weight_packed"] = codes
            t[f"m.{p}.weight_scale"] = sc.view(torch.uint8)
            t[f"m.{p}.weight_global_scale"] = torch.tensor([1.0 / mul], dtype=torch.float32)
            t[f"m.{p}.input_global_scale"] = torch.tensor([1.0], dtype=torch.float32)
        else:
            t[f"m.{p}.weight"] = codes
            t[f"m.{p}.weight_scale"] = sc
            t[f"m.{p}.weight_scale_2"] = torch.tensor(mul, dtype=torch.float32)
            t[f"m.{p}.input_scale"] = torch.tensor(1.0, dtype=torch.float32)
    tensors = _roundtrip(tmp_path, t)
    m, lay = LD.build_linear(q, "m.gate_up_proj", K, 2 * I, tensors, parts=["m.gate_proj", "m.up_proj"], device="cpu")
    assert isinstance(m, M_.NvFp4LinearMethod)
    glob = lay._global_op.view(torch.float32)
    want = torch.cat([torch.full((I,), float(torch.tensor(1.0) / torch.tensor(1.0 / 0.001))
                                 if producer == "compressed-tensors" else float(torch.tensor(0.001))),
                      torch.full((I,), float(torch.tensor(1.0) / torch.tensor(1.0 / 0.002))
                                 if producer == "compressed-tensors" else float(torch.tensor(0.002)))])
    assert torch.equal(glob, want)
    assert lay._scales_op.shape == (K // 16, 2 * I)


def test_gptq_experts_stacked(tmp_path):
    E, H, I, g = 4, 256, 128, 128
    q = Q(method="gptq", bits=4, group_size=g, sym=False)
    gen = synth.gen(6)
    t = {}
    for e in range(E):
        for p, (n, k) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            t[f"x.{e}.{p}.qweight"] = _rand_i32((k // 8, n), gen)
            t[f"x.{e}.{p}.scales"] = (torch.rand(k // g, n, generator=gen) * 0.02).to(torch.float16)
            # GPTQ stores zero - 1: nibbles 0..14
            z = torch.randint(0, 15, (k // g, n), generator=gen, dtype=torch.int32)
            t[f"x.{e}.{p}.qzeros"] = synth.pack_rows(z)
    tensors = _roundtrip(tmp_path, t)
    mm, w13, w2 = LD.build_experts(q, "x", E, H, I, tensors, device="cpu")
    for e in range(E):
        ops = [K_.gptq_to_op_layout(t[f"x.{e}.{p}.qweight"], t[f"x.{e}.{p}.scales"], t[f"x.{e}.{p}.qzeros"])
               for p in ("gate_proj", "up_proj")]
        assert torch.equal(w13._scales_op[e], torch.cat([o[1] for o in ops], dim=1))
        assert torch.equal(w13._zeros_op[e], torch.cat([o[2] for o in ops], dim=1))
        d = K_.gptq_to_op_layout(t[f"x.{e}.down_proj.qweight"], t[f"x.{e}.down_proj.scales"], t[f"x.{e}.down_proj.qzeros"])
        assert torch.equal(w2._scales_op[e], d[1])


# ------------------------------------------------------------------------------------ AMD Quark
def _quark(dtype, sfmt, **extra):
    w = {"dtype": dtype, "scale_format": sfmt, "group_size": extra.pop("group_size", 32), "is_dynamic": False}
    w.update(extra.pop("weight_extra", {}))
    d = {"quant_method": "quark", "global_quant_config": {"weight": w,
                                                          "input_tensors": {"dtype": "fp4", "is_dynamic": False}},
         "exclude": ["lm_head", "model.language_model.layers.0.mlp.gate.weight", "mtp.layers.0.mlp.gate_proj.weight",
                     "model.layers.1.self_attn.q_proj.bias", "model.layers.2.mlp.up_proj.weight_scale"],
         "export": {"pack_method": "reorder"}}
    d.update(extra)
    return {"quantization_config": d}


def test_from_hf_quark_formats_and_exclude_suffixes():
    """Quark (python/minisgl/quant/config.py:228-293): the (dtype, scale_format) pair names the
    format; exclude entries name tensors, cut to their module (else `mtp...gate_proj.weight` would
    match no module and the unquantized tensor would load as a quantized layer)."""
    mx = Q.from_hf(_quark("fp4", "e8m0"))
    assert mx.is_compressed_tensors and mx.weight_is_e2m1 and not mx.is_nvfp4 and mx.group_size == 32
    assert mx.ct_format == "mxfp4-pack-quantized" and mx.act_type is None
    assert mx.ignore == ("lm_head", "model.layers.0.mlp.gate", "mtp.layers.0.mlp.gate_proj",
                         "model.layers.1.self_attn.q_proj", "model.layers.2.mlp.up_proj")
    assert mx.for_module("mtp.layers.0.mlp.gate_proj") is None
    assert mx.for_module("model.layers.0.mlp.gate") is None
    assert mx.for_module("model.layers.3.mlp.gate_proj") is mx
    assert isinstance(M_.create_linear_method(mx), M_.MxFp4LinearMethod)
    nv = Q.from_hf(_quark("fp4", "e4m3", group_size=16))
    assert nv.is_nvfp4 and nv.group_size == 16 and isinstance(M_.create_linear_method(nv), M_.NvFp4LinearMethod)
    f8 = Q.from_hf(_quark("fp8_e4m3", "float"))
    assert f8.is_fp8_w8a8 and f8.ct_format == "float-quantized"
    assert Q.from_hf(_quark("fp8_e4m3", "")).is_fp8_w8a8


@pytest.mark.parametrize("bad", [
    dict(dtype="int4", sfmt="float"),                          # pair outside the closed table
    dict(dtype="fp4", sfmt="fp16"),
    dict(dtype="fp4", sfmt="e8m0", weight_extra={"is_dynamic": True}),
    dict(dtype="fp4", sfmt="e8m0", layer_quant_config={"model.layers.0.mlp.down_proj": {"weight": {"dtype": "fp8_e4m3"}}}),
    dict(dtype="fp4", sfmt="e8m0", layer_type_quant_config={"Linear": {}}),
    dict(dtype="fp4", sfmt="e8m0", export={"pack_method": "order"}),
])
def test_from_hf_quark_refusals(bad):
    """Each refusal returns None (the header is not served) instead of a scheme that would load
    and compute wrong numbers: dynamic weight quant, per-layer overrides, an unknown packing."""
    bad = dict(bad)
    assert Q.from_hf(_quark(bad.pop("dtype"), bad.pop("sfmt"), **bad)) is None


def test_quark_mxfp4_layer_from_safetensors(tmp_path):
    """A Quark MXFP4 checkpoint names the packed codes `weight` (uint8) beside `weight_scale`; the
    loader builds the same layer as from the compressed-tensors names."""
    K, I = 256, 32
    q = Q.from_hf(_quark("fp4", "e8m0"))
    gen = synth.gen(8)
    quark, ct = {}, {}
    for p in ("gate_proj", "up_proj"):
        codes = torch.randint(0, 256, (I, K // 2), generator=gen, dtype=torch.int32).to(torch.uint8)
        sc = torch.randint(119, 128, (I, K // 32), generator=gen, dtype=torch.int32).to(torch.uint8)
        quark[f"model.layers.3.mlp.{p}.weight"] = codes
        quark[f"model.layers.3.mlp.{p}.weight_scale"] = sc
        ct[f"model.layers.3.mlp.{p}.weight_packed"] = codes
        ct[f"model.layers.3.mlp.{p}.weight_scale"] = sc
    parts = ["model.layers.3.mlp.gate_proj", "model.layers.3.mlp.up_proj"]
    mq, lq = LD.build_linear(q, "model.layers.3.mlp.gate_up_proj", K, 2 * I, _roundtrip(tmp_path, quark), parts=parts,
                             device="cpu")
    mc, lc = LD.build_linear(q, "model.layers.3.mlp.gate_up_proj", K, 2 * I, ct, parts=parts, device="cpu")
    assert isinstance(mq, M_.MxFp4LinearMethod)
    dq, dc = LD._declared(lq), LD._declared(lc)
    assert dq.keys() == dc.keys() and all(torch.equal(dq[k], dc[k]) for k in dq)
    # a full-precision `weight` is never taken for the packed codes
    with pytest.raises(KeyError, match="weight_packed"):
        LD.build_linear(q, "m", K, I, {"m.weight": torch.randn(I, K).to(torch.bfloat16),
                                       "m.weight_scale": torch.zeros(I, K // 32, dtype=torch.uint8)}, device="cpu")
