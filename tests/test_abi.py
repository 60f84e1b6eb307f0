"""C ABI surface and host-side refusal behaviour -- no kernel launches, runs without a GPU."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from conftest import REPO, pkg

HEADER = REPO / "include" / "w4a8_mi355x.h"
HEADERS = sorted((REPO / "include").glob("*.h"))


def _header_text() -> str:
    return "\n".join(h.read_text() for h in HEADERS)


def _declared() -> list[str]:
    text = _header_text()
    return sorted(set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(w4a(?:8|16)_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    abi = pkg("_abi")
    if not abi.lib_path().exists():
        pkg().__class__  # noqa: B018
        import importlib.util

        spec = importlib.util.spec_from_file_location("w4a8_build", REPO / "minisglang-rdna4_amd" / "build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return abi.load()


def test_header_declares_the_bound_surface():
    abi = pkg("_abi")
    assert _declared() == sorted(abi.SIGNATURES)


def _declared_params() -> dict[str, list[str]]:
    """name -> parameter type list, parsed from the header's prototypes."""
    text = re.sub(r"/\*.*?\*/", "", _header_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(w4a(?:8|16)_\w+)\s*\(([^)]*)\)\s*;", text, re.M):
        params = [p.strip() for p in m.group(2).replace("\n", " ").split(",") if p.strip()]
        if params == ["void"]:
            params = []
        out[m.group(1)] = [re.sub(r"\s*\b\w+$", "", p) for p in params]
    return out


def _ctype_of(decl: str):
    decl = decl.replace("const ", "").strip()
    if "*" in decl:
        return ctypes.c_void_p if decl not in ("char*", "char *") else ctypes.c_char_p
    return {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "float": ctypes.c_float}[decl]


def test_bindings_match_header_prototypes():
    """Each ctypes signature has the header's parameter count and kinds (pointer / int / int64 / float)."""
    abi = pkg("_abi")
    protos = _declared_params()
    assert sorted(protos) == _declared()
    for name, params in protos.items():
        _, argtypes = abi.SIGNATURES[name]
        assert len(argtypes) == len(params), f"{name}: binding has {len(argtypes)} args, header {len(params)}"
        for i, (a, d) in enumerate(zip(argtypes, params)):
            assert a == _ctype_of(d), f"{name} arg {i}: binding {a}, header {d!r}"


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(str(pkg("_abi").lib_path()))
    for name in _declared():
        assert hasattr(raw, name), f"{name} declared in include/ but not exported"
    # the revision the header declares is the one the library reports
    assert lib.w4a8_abi_version() == int(re.search(r"#define W4A8_ABI_VERSION (\d+)", HEADER.read_text()).group(1)) == 5


def test_host_validation_rejects_before_launch(lib):
    # N not a multiple of 16: refused on the host with a message, no device pointer touched
    rc = lib.w4a8_gemm(None, 128, None, 1, None, 24, 128, None, 0, None, 0, 128, None, 0, 24, 0, None, 0, 0, None)
    assert rc == 1 and b"multiple of 16" in lib.w4a8_last_error()
    rc = lib.w4a8_gemm(None, 128, None, 1, None, 32, 128, None, 1, None, 0, 32, None, 0, 32, 0, None, 0, 0, None)
    assert rc == 1 and b"E8M0" in lib.w4a8_last_error()
    rc = lib.w4a8_gemm(None, 256, None, 1, None, 32, 256, None, 0, None, 0, 48, None, 0, 32, 0, None, 0, 0, None)
    assert rc == 2 and b"group_size" in lib.w4a8_last_error()
    rc = lib.w4a8_moe_align(None, 8, 600, 16, 10000, None, None, None, None, None)
    assert rc == 2 and b"num_experts" in lib.w4a8_last_error()
    rc = lib.w4a8_moe_align(None, 8, 8, 16, 10, None, None, None, None, None)
    assert rc == 1 and b"capacity" in lib.w4a8_last_error()
    # the grouped kernels index slots and padded rows in 32 bits: 2^31 of either is refused
    rc = lib.w4a8_moe_align(None, 8, 8, 16, 1 << 31, None, None, None, None, None)
    assert rc == 1 and b"2^31" in lib.w4a8_last_error()
    moe_gemm = lambda numel, top_k, P: lib.w4a8_moe_gemm(  # noqa: E731
        None, 256, None, 1, None, None, None, numel, top_k, 16, P, None, 8, 64, 256, None, 0, None, 0, 128, None, 0,
        64, 0, None, 0, 0, None)
    assert moe_gemm(8, 2, 1 << 31) == 1 and b"2^31" in lib.w4a8_last_error()
    assert moe_gemm(1 << 31, 2, 4096) == 1 and b"2^31" in lib.w4a8_last_error()
    assert moe_gemm(8, 0, 4096) == 1 and b"top_k" in lib.w4a8_last_error()
    assert lib.w4a8_tile_bytes(32, 256) == 2 * 2 * 1024
    assert lib.w4a8_tile_bytes(32, 160) == 2 * 2 * 1024
    assert lib.w4a8_moe_padded_capacity(8, 128, 16) == 8 + 129 * 15
    # one block per slot: no more slots than experts
    P = lib.w4a8_moe_padded_capacity(16, 8, 16)
    rc = lib.w4a8_moe_route_slots(None, 0, 2, 8, 8, 1, 16, P, None, None, None, None, None, None, None, 0, 0, 0, None,
                                  0, None, None)
    assert rc == 1 and b"slots" in lib.w4a8_last_error()


# ------------------------------------------------------------------------ provider refusals
def _dense_args(M=4, K=256, N=64, g=128):
    x = torch.randn(M, K).to(torch.bfloat16)
    w = torch.zeros((N, K // 8), dtype=torch.int32)
    s = torch.ones((K // g, N), dtype=torch.float16)
    return x, w, s


def test_half_producer_pair_refused_loudly():
    K_ = pkg("quant.kernels")
    x, w, s = _dense_args()
    q = torch.zeros(x.shape, dtype=torch.uint8)
    sc = torch.ones(x.shape[0])
    with pytest.raises(RuntimeError, match="TOGETHER"):
        K_.w4a8_linear(x, w, s, None, 128, x_fp8=q)
    with pytest.raises(RuntimeError, match="TOGETHER"):
        K_.w4a8_linear(x, w, s, None, 128, act_scales=sc)
    with pytest.raises(RuntimeError, match="x_fp8 must be"):
        K_.w4a8_linear(x, w, s, None, 128, x_fp8=q[:, :128].contiguous(), act_scales=sc)
    with pytest.raises(RuntimeError, match="in-prologue"):
        K_.w4a8_linear(x, w, s, None, 128, kernel="prefill_wmma", x_fp8=q, act_scales=sc)


def test_scale_layout_and_format_refusals():
    K_ = pkg("quant.kernels")
    x, w, s = _dense_args()
    with pytest.raises(AssertionError, match="GROUP-major"):
        K_.w4a8_linear(x, w, s.t().contiguous(), None, 128)
    with pytest.raises(TypeError, match="E8M0"):
        K_.w4a8_linear(x, w, torch.zeros((256 // 32, 64), dtype=torch.uint8), None, 32)
    with pytest.raises(AssertionError, match="symmetric"):
        K_.w4a8_linear(x, w, torch.ones((8, 64), dtype=torch.float16), torch.zeros((8, 8), dtype=torch.int32), 32,
                       weight_is_e2m1=True)
    # one-byte scales with the zeros slot populated are NVFP4: the slot must hold the (N,) f32 global
    with pytest.raises(AssertionError, match="NVFP4 global"):
        K_.w4a8_linear(x, w, torch.zeros((8, 64), dtype=torch.uint8), torch.zeros((8, 8), dtype=torch.int32), 32,
                       weight_is_e2m1=True)
    with pytest.raises(AssertionError, match="REQUIRE"):
        K_.w4a8_linear(x, w, torch.zeros((16, 64), dtype=torch.float8_e4m3fn), None, 16, weight_is_e2m1=True)


# tests/mxfp4_moe_scale_guard_test.py:27-58 restated against this provider
E, N, K, G = 4, 64, 256, 32


def _w():
    return torch.zeros((E, N, K // 8), dtype=torch.int32)


def test_moe_scale_guard_accepts_mxfp4_e8m0():
    pkg("quant.kernels")._check_moe_scale_pair(_w(), torch.zeros((E, K // G, N), dtype=torch.uint8), None, "w13")


def test_moe_scale_guard_refuses_e4m3_without_global():
    with pytest.raises(AssertionError, match="REQUIRE the per-output-channel f32 global"):
        pkg("quant.kernels")._check_moe_scale_pair(
            _w(), torch.zeros((E, K // 16, N), dtype=torch.float8_e4m3fn), None, "w13")


def test_moe_scale_guard_validates_global():
    chk = pkg("quant.kernels")._check_moe_scale_pair
    chk(_w(), torch.zeros((E, K // 16, N), dtype=torch.uint8), torch.zeros((E, N), dtype=torch.int32), "w13")
    with pytest.raises(AssertionError):
        chk(_w(), torch.zeros((E, K // 16, N), dtype=torch.uint8), torch.zeros((E, N), dtype=torch.float32), "w13")


def test_moe_scale_guard_fp16_and_unknown():
    chk = pkg("quant.kernels")._check_moe_scale_pair
    chk(_w(), torch.zeros((E, K // G, N), dtype=torch.float16), None, "w13")
    with pytest.raises(AssertionError, match="scales must be"):
        chk(_w(), torch.zeros((E, K // G, N), dtype=torch.bfloat16), None, "w13")
    with pytest.raises(AssertionError, match="2-D zeros"):
        chk(_w(), torch.zeros((E, K // G, N), dtype=torch.float16), torch.zeros((E, N), dtype=torch.int32), "w13")


def test_moe_block_m_policy():
    bm = pkg("quant.kernels")._moe_block_m
    # BASELINE MoE config: E=128, top-8
    assert [bm(T, 128, 8, flag_gemm1=True) for T in (1, 16, 256, 4096)] == [16, 16, 64, 128]
    assert bm(64, 32, 4) == 16 and bm(2048, 32, 4) == 128


def test_moe_block_m_auto_policy(monkeypatch):
    """w4a8_moe's own choice: 16-row GEMV blocks up to 32 routed rows per expert, 64-row tiles up to
    44, 128-row tiles above; MINISGL_MOE_BLOCK_M forces a value as in the reference."""
    auto = pkg("quant.kernels")._moe_block_m_auto
    monkeypatch.delenv("MINISGL_MOE_BLOCK_M", raising=False)
    assert [auto(T, 128, 8) for T in (1, 16, 256, 512, 576, 640, 704, 768, 1024, 4096)] == \
        [16, 16, 16, 16, 64, 64, 64, 128, 128, 128]
    assert auto(64, 32, 4) == 16 and auto(2048, 32, 4) == 128
    monkeypatch.setenv("MINISGL_MOE_BLOCK_M", "64")
    assert auto(4096, 128, 8) == 64


def test_pick_dense_kernel():
    pick = pkg("quant.kernels")._pick_dense_kernel
    assert pick(1, k=4096) == "decode_gemv" and pick(16, k=4096) == "decode_gemv"
    assert pick(17, k=4096) == "wmma_tiled_tuned" and pick(8, k=4100) == "wmma_tiled_tuned"
    assert pick(16, weight_is_e2m1=True, group_size=32, k=8192) == "decode_gemv"


def test_linear_launch_count(lib):
    """Launches per w4a8_linear call (host-only planner query): the configs[1] step's calls are single
    launches (the GEMV quantizes its rows) except the two 14336-wide down projections at 8 and 16
    rows; prefill calls and sub-tile groups take the act-quant launch first."""
    step = {}
    for K, N in [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)]:
        for M in (1, 2, 4, 8, 16):
            step[(K, N, M)] = lib.w4a8_linear_launch_count(M, N, K, 0, 0, 0, 0, 128, 0, 0)
    assert all(v in (1, 2) for v in step.values())
    assert [k for k, v in step.items() if v == 2] == [(4096, 6144, 16), (4096, 4096, 16), (14336, 4096, 8),
                                                      (14336, 4096, 16)]
    assert sum(step.values()) == 24
    assert lib.w4a8_linear_launch_count(0, 4096, 4096, 0, 0, 0, 0, 128, 0, 0) == 0
    assert lib.w4a8_linear_launch_count(17, 4096, 4096, 0, 0, 0, 0, 128, 0, 0) == 2
    assert lib.w4a8_linear_launch_count(4, 4096, 4096, 1, 0, 1, 0, 128, 1, 0) == 1
    assert lib.w4a8_linear_launch_count(4, 4096, 4096, 0, 0, 1, 0, 32, 0, 0) == 2
    assert lib.w4a8_linear_launch_count(4, 24, 128, 0, 0, 0, 0, 128, 0, 0) == -1
    assert b"multiple of 16" in lib.w4a8_last_error()
    # prefill: one quant launch (row-major, or straight into the GEMM's operand order) and the GEMM
    for M, N, zeros, e2 in ((2048, 28672, 0, 0), (1023, 28672, 0, 0), (2048, 6144, 0, 0), (2048, 28672, 1, 0),
                            (2048, 28672, 0, 1)):
        assert lib.w4a8_linear_launch_count(M, N, 4096, 0, e2, zeros, e2, 32 if e2 else 128, 0, 0) == 2
