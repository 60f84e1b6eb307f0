"""The two integration routes of INTEGRATION.md, exercised as written.

Option A: alias.install() makes the reference's module names resolve to this package. Option B: the
ctypes binding printed in INTEGRATION.md is executed against the built library; on the CPU its
argument tables must match the exported symbols, and on the GPU its mmq_fp8_gemm /
mmq_fp8_gemm_silu (the signatures of the reference's fp8_wmma ops) must give this package's
w4a8_linear / w4a8_linear_silu bits exactly, for int4 (asymmetric), MXFP4 and NVFP4 weights, with
and without the producer pair.
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


def _stub_source() -> str:
    text = (REPO / "INTEGRATION.md").read_text()
    m = re.search(r"```python\n(# python/minisgl/quant/_w4a8_mi355x\.py.*?)```", text, re.S)
    assert m, "INTEGRATION.md lost its Option B binding block"
    return m.group(1)


@pytest.fixture(scope="module")
def stub():
    if not LIB.exists():
        pytest.skip("library not built")
    os.environ["W4A8_MI355X_LIB"] = str(LIB)
    mod = types.ModuleType("_w4a8_mi355x_stub")
    exec(compile(_stub_source(), "INTEGRATION.md:_w4a8_mi355x.py", "exec"), mod.__dict__)
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
