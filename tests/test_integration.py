"""The two integration routes of INTEGRATION.md, exercised as written.

Option A: alias.install() makes the reference's module names resolve to this package. Option B: the
two ctypes binding blocks printed in INTEGRATION.md (dense, MoE) are executed against the built
library; on the CPU their argument tables must match the exported symbols. On the GPU the dense
block's mmq_fp8_gemm / mmq_fp8_gemm_silu (the signatures of the reference's fp8_wmma ops) must give
this package's w4a8_linear / w4a8_linear_silu bits exactly, for int4 (asymmetric), MXFP4 and NVFP4
weights, with and without the producer pair; the MoE block runs the reference's own w4a8_moe call
sequences and must give this package's _moe_forward bits exactly.
"""
import importlib
import os
import re
import sys
import types
from pathlib import Path

import pytest
import torch

import synth
from conftest import pkg

REPO = Path(__file__).resolve().parents[1]
LIB = REPO / "minisglang-rdna4_amd" / "_lib" / "libw4a8_mi355x.so"


def _stub_source(name: str = "_w4a8_mi355x") -> str:
    text = (REPO / "INTEGRATION.md").read_text()
    m = re.search(r"```python\n(# python/minisgl/quant/" + name + r"\.py.*?)```", text, re.S)
    assert m, f"INTEGRATION.md lost its Option B binding block {name}"
    return m.group(1)


@pytest.fixture(scope="module")
def stub():
    if not LIB.exists():
        pytest.skip("library not built")
    os.environ["W4A8_MI355X_LIB"] = str(LIB)
    mod = types.ModuleType("_w4a8_mi355x_stub")
    exec(compile(_stub_source(), "INTEGRATION.md:_w4a8_mi355x.py", "exec"), mod.__dict__)
    return mod


@pytest.fixture(scope="module")
def moe_stub(stub):
    """The MoE binding block, executed with the dense block importable under the reference's module
    name (minisgl.quant._w4a8_mi355x), as it would be installed there."""
    names = ("minisgl", "minisgl.quant", "minisgl.quant._w4a8_mi355x")
    saved = {k: sys.modules.get(k) for k in names}
    root, quant = types.ModuleType("minisgl"), types.ModuleType("minisgl.quant")
    root.__path__, quant.__path__ = [], []
    sys.modules.update({"minisgl": root, "minisgl.quant": quant, "minisgl.quant._w4a8_mi355x": stub})
    try:
        mod = types.ModuleType("_w4a8_mi355x_moe_stub")
        exec(compile(_stub_source("_w4a8_mi355x_moe"), "INTEGRATION.md:_w4a8_mi355x_moe.py", "exec"), mod.__dict__)
    finally:
        for k, v in saved.items():
            if v is None:
                sys.modules.pop(k, None)
            else:
                sys.modules[k] = v
    return mod


def test_alias_install_resolves_reference_names():
    al = pkg("alias")
    saved = {k: v for k, v in sys.modules.items() if k == "minisgl" or k.startswith("minisgl.")}
    try:
        for k in list(saved):
            del sys.modules[k]
        al.install()
        from minisgl.quant import kernels  # noqa: the reference's import line
        import minisgl.layers.moe as moe
        import minisgl.quant.method as method

        assert kernels is pkg("quant.kernels") and moe is pkg("layers.moe") and method is pkg("quant.method")
        assert callable(kernels.w4a8_linear) and callable(kernels.w4a8_moe) and callable(kernels.w4a16_moe)
        assert callable(moe.create_moe_quant_method) and callable(method.create_linear_method)
        with pytest.raises(ImportError):
            importlib.import_module("minisgl.engine")
    finally:
        for k in [k for k in sys.modules if k == "minisgl" or k.startswith("minisgl.")]:
            del sys.modules[k]
        sys.modules.update(saved)


def test_stub_binds_exported_symbols(stub):
    """The stub's argtypes agree with the package's own signature table for every symbol it binds."""
    sig = pkg("_abi").SIGNATURES
    for name in ("w4a8_tile_bytes", "w4a8_repack_weights", "w4a8_linear_workspace_bytes",
                 "w4a8_gemm_workspace_bytes", "w4a8_gemm", "w4a8_linear"):
        fn = getattr(stub._lib, name)
        assert list(fn.argtypes) == list(sig[name][1]), name
        assert fn.restype == sig[name][0], name


def test_moe_stub_binds_exported_symbols(moe_stub):
    sig = pkg("_abi").SIGNATURES
    for name in ("w4a8_moe_padded_capacity", "w4a8_moe_route_align", "w4a8_moe_align", "w4a8_act_quant",
                 "w4a8_moe_gemm_workspace_bytes", "w4a8_moe_gemm", "w4a8_moe_combine",
                 "w4a8_moe_gemm2_combine_supported", "w4a8_moe_gemm2_combine"):
        fn = getattr(moe_stub._lib, name)
        assert list(fn.argtypes) == list(sig[name][1]), name
        assert fn.restype == sig[name][0], name


def _weights(fmt, N, K, seed):
    if fmt == "asym":
        w, s, z = synth.int4_weight(N, K, 128, seed=seed, asym=True, scale_floor=1e-4)
        return w, s, z, False, 128
    if fmt == "mxfp4":
        w, s = synth.mxfp4_weight(N, K, seed=seed)
        return w, s, None, True, 32
    w, s, g = synth.nvfp4_weight(N, K, seed=seed)
    return w, s, g, True, 16


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["asym", "mxfp4", "nvfp4"])
def test_stub_matches_operator(stub, kernels, dev, fmt):
    K, N = 1024, 512
    w, s, z, e2, g = _weights(fmt, N, K, seed=len(fmt))
    wd, sd, zd = w.to(dev), s.to(dev), None if z is None else z.to(dev)
    tiles = stub.repack(wd, e2)
    assert torch.equal(tiles, kernels.repack_w4(wd, weight_is_e2m1=e2))
    for M in (1, 5, 16, 64):
        x = synth.activations(M, K, seed=M + 3).to(dev)
        ref = kernels.w4a8_linear(x, tiles, sd, zd, g, weight_is_e2m1=e2)
        got_op = stub.mmq_fp8_gemm(x, wd, sd, w_zeros=zd, weight_is_e2m1=e2)
        got_tiles = stub.mmq_fp8_gemm(x, tiles, sd, w_zeros=zd, weight_is_e2m1=e2)
        q, a = kernels.act_quant(x)
        ref_pair = kernels.w4a8_linear(x, tiles, sd, zd, g, weight_is_e2m1=e2, x_fp8=q, act_scales=a)
        got_pair = stub.mmq_fp8_gemm(x, tiles, sd, w_zeros=zd, weight_is_e2m1=e2, x_fp8=q, act_scales=a)
        torch.cuda.synchronize()
        assert torch.equal(got_op, ref) and torch.equal(got_tiles, ref), f"{fmt} M={M}"
        assert torch.equal(got_pair, ref_pair), f"{fmt} M={M} producer pair"
        if M <= 16:
            ref_s = kernels.w4a8_linear_silu(x, tiles, sd, zd, g, weight_is_e2m1=e2)
            got_s = stub.mmq_fp8_gemm_silu(x, tiles, sd, w_zeros=zd, weight_is_e2m1=e2)
            torch.cuda.synchronize()
            assert torch.equal(got_s, ref_s), f"{fmt} M={M} silu"


def _moe_experts(fmt, e, h, i, seed):
    from test_gpu_moe import _fmt_experts

    return _fmt_experts(fmt, e, h, i, seed)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["sym", "asym", "mxfp4", "nvfp4"])
@pytest.mark.parametrize("T,bm", [(3, 16), (48, 16), (300, 64)])
def test_moe_stub_runs_reference_sequence(moe_stub, kernels, dev, monkeypatch, fmt, T, bm):
    """The reference's w4a8_moe sequence on the MoE binding (python/minisgl/quant/kernels.py:686-882):
    moe_route_align (or moe_align on given ids), mmq_fp8_moe_gemm1_silu, then either the decode
    mmq_fp8_moe_gemm2_gather_reduce or mmq_fp8_moe_gemm over the identity rows (top_k = 1) and
    mmq_fp8_moe_gather_reduce; each against this package's _moe_forward on the same route, bit for
    bit (the fused decode form against _moe_forward with unrounded gemm2 rows, the unfused form
    against it with rows in x's dtype, as the reference hands them over on each path)."""
    e, h, i, k = 32, 1024, 768, 8
    w13, s13, z13, w2, s2, z2, e2 = _moe_experts(fmt, e, h, i, seed=600 + T)
    d = lambda t: None if t is None else t.to(dev)
    t13 = kernels.repack_w4(w13.to(dev), weight_is_e2m1=e2)
    t2 = kernels.repack_w4(w2.to(dev), weight_is_e2m1=e2)
    x = synth.activations(T, h, seed=610 + T).to(dev)
    lg = synth.router_logits(T, e, seed=611 + T).to(dev)
    # the route: the binding's moe_route_align against the package's router, ids and weights exactly
    tw_s, ids_s, sorted_s, experts_s, ntp_s = moe_stub.moe_route_align(lg, k, True, e, bm)
    tw, ids = kernels._moe_route(lg, k, True, e)
    torch.cuda.synchronize()
    assert torch.equal(ids_s, ids) and torch.equal(tw_s, tw)
    sorted_ids, expert_ids, ntp = moe_stub.moe_align(ids, e, bm)
    kern = "gemv" if bm < 64 else None
    buf2 = moe_stub.mmq_fp8_moe_gemm1_silu(x, t13, d(s13), sorted_ids, expert_ids, ntp, k, bm, kernel=kern,
                                           w_zeros=d(z13), weight_is_e2m1=e2)
    tw_flat = tw.reshape(-1)
    ident = torch.arange(sorted_ids.numel(), dtype=torch.int32, device=dev)
    out2 = moe_stub.mmq_fp8_moe_gemm(buf2, t2, d(s2), ident, expert_ids, ntp, 1, bm, kernel=kern, w_zeros=d(z2),
                                     weight_is_e2m1=e2)
    unfused = moe_stub.mmq_fp8_moe_gather_reduce(out2, sorted_ids, tw_flat, ntp, k).to(x.dtype)
    args = (t13, d(s13), d(z13), t2, d(s2), d(z2), None, k, True)
    kw = dict(topk_weights=tw, topk_ids=ids, block_m=bm, weight_is_e2m1=e2)
    monkeypatch.setattr(kernels, "_MOE_G2FUSE", False)
    ref_rounded = kernels._moe_forward(x, *args, y2_dtype=x.dtype, **kw)
    torch.cuda.synchronize()
    rows = torch.nonzero(sorted_ids < T * k).flatten()  # padded rows that hold a slot
    assert torch.equal(buf2[rows], ref_rounded["buf2"][rows]), f"{fmt} T={T} bm={bm}: gemm1 rows differ"
    assert torch.equal(unfused, ref_rounded["out"]), f"{fmt} T={T} bm={bm}: unfused sequence differs"
    if bm < 64:
        fused = moe_stub.mmq_fp8_moe_gemm2_gather_reduce(buf2, t2, d(s2), sorted_ids, expert_ids, ntp, tw_flat, k, bm,
                                                         w_zeros=d(z2), weight_is_e2m1=e2).to(x.dtype)
        ref_f32 = kernels._moe_forward(x, *args, y2_dtype=torch.float32, **kw)
        torch.cuda.synchronize()
        assert torch.equal(fused, ref_f32["out"]), f"{fmt} T={T} bm={bm}: decode gemm2_gather_reduce differs"
