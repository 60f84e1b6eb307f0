"""CPU oracle for the W4A8 path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and
only as the checker (or the timed CPU baseline), never as the thing measured or shipped. The
product package never imports it.

The arithmetic lives in w4a8_oracle.c (a restatement of the reference's formulas, with file:line
citations); this module binds it with ctypes and adds numpy helpers. Parity status per function is
recorded in the C file's header; the pins are exercised in tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libw4a8_oracle.so"

E2M1_LUT = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                     -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float64)

_lib = None


def build() -> Path:
    r = subprocess.run(["make", "-s", "-C", str(HERE)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        vp, i64, ci, f = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.w4o_f32_to_e4m3.restype = ctypes.c_uint8
        L.w4o_f32_to_e4m3.argtypes = [f]
        L.w4o_e4m3_to_f32.restype = f
        L.w4o_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.w4o_act_quant.restype = None
        L.w4o_act_quant.argtypes = [vp, ci, i64, i64, i64, vp, vp]
        L.w4o_gemm.restype = None
        L.w4o_gemm.argtypes = [vp, vp, i64, i64, vp, i64, vp, ci, vp, ci, i64, vp]
        L.w4o_dequant.restype = None
        L.w4o_dequant.argtypes = [vp, i64, i64, vp, ci, vp, ci, i64, vp]
        L.w4o_moe_route.restype = None
        L.w4o_moe_route.argtypes = [vp, i64, i64, i64, ci, vp, vp]
        L.w4o_moe_align.restype = i64
        L.w4o_moe_align.argtypes = [vp, i64, i64, i64, vp, vp, vp, vp]
        L.w4o_moe_forward.restype = None
        L.w4o_moe_forward.argtypes = [vp, ci, i64, i64, i64, i64, i64, vp, vp, vp, ctypes.c_int32, i64,
                                      vp, vp, vp, vp, vp, vp, ci, ci, i64, i64, vp, vp, ci]
        L.w4o_w4a16_moe_forward.restype = None
        L.w4o_w4a16_moe_forward.argtypes = [vp, ci, i64, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, ci, ci,
                                            i64, i64, vp, vp]
        L.w4o_rms_norm.restype = None
        L.w4o_rms_norm.argtypes = [vp, vp, vp, ci, f, ci, i64, i64, vp]
        L.w4o_act_split.restype = None
        L.w4o_act_split.argtypes = [vp, ci, i64, i64, vp, vp]
        L.w4o_silu_mul.restype = ctypes.c_uint16
        L.w4o_silu_mul.argtypes = [ctypes.c_double, ctypes.c_double, ci]
        L.w4o_bf16_to_f32.restype = f
        L.w4o_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.w4o_f32_to_bf16.restype = ctypes.c_uint16
        L.w4o_f32_to_bf16.argtypes = [f]
        L.w4o_f16_to_f32.restype = f
        L.w4o_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.w4o_f32_to_f16.restype = ctypes.c_uint16
        L.w4o_f32_to_f16.argtypes = [f]
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- scalar / vector codecs
def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """Closed-form OCP e4m3fn decode (1-4-3, bias 7, S.1111.111 = NaN)."""
    c = np.asarray(codes).astype(np.int64)
    s, e, m = c >> 7, (c >> 3) & 15, c & 7
    v = np.where(e == 0, m * 2.0 ** -9, (8 + m) * 2.0 ** (e - 10))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return np.where(s == 1, -v, v)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    L = lib()
    flat = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.fromiter((L.w4o_f32_to_e4m3(float(v)) for v in flat), dtype=np.uint8, count=flat.size)
    return out.reshape(np.shape(x))


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns (RNE)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- kernels
def act_quant(x_bits: np.ndarray, dtype: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """x_bits: (M, K) uint16 bf16 (dtype 0) / fp16 (dtype 1) patterns -> (codes (M,K) u8, scales (M,) f32)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    M, K = x.shape
    q = np.empty((M, K), dtype=np.uint8)
    s = np.empty((M,), dtype=np.float32)
    lib().w4o_act_quant(_p(x), dtype, M, K, K, _p(q), _p(s))
    return q, s


def _scales_arg(scales: np.ndarray, zeros, nvfp4: bool):
    """(scale buffer, format code, zeros/global buffer). NVFP4: e4m3 block-scale bytes (uint8) with the
    per-channel f32 global multiplier in the zeros slot (f32 or its int32 bit pattern)."""
    if nvfp4:
        sc, fmt = np.ascontiguousarray(scales, dtype=np.uint8), 2
        z = np.ascontiguousarray(np.asarray(zeros).view(np.int32) if np.asarray(zeros).dtype == np.float32
                                 else zeros, dtype=np.int32)
        return sc, fmt, z
    if scales.dtype == np.float16:
        sc, fmt = np.ascontiguousarray(scales).view(np.uint16), 0
    else:
        sc, fmt = np.ascontiguousarray(scales, dtype=np.uint8), 1
    return sc, fmt, None if zeros is None else np.ascontiguousarray(zeros, dtype=np.int32)


def gemm(xq: np.ndarray, xs: np.ndarray, w_packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray | None,
         group: int, e2m1: bool = False, nvfp4: bool = False) -> np.ndarray:
    """f64 y[m,n] = s_m * sum_g scale[g,n] * sum_{k in g} e4m3(q[m,k]) * w(n,k).
    scales: (G,N) float16 (passed as its uint16 bits), uint8 E8M0, or (nvfp4) e4m3 bytes with the
    (N,) f32 global in zeros."""
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    w = np.ascontiguousarray(w_packed, dtype=np.int32)
    M, K = xq.shape
    N = w.shape[0]
    sc, fmt, z = _scales_arg(scales, zeros, nvfp4)
    out = np.empty((M, N), dtype=np.float64)
    lib().w4o_gemm(_p(xq), _p(xs), M, K, _p(w), N, _p(sc), fmt, _p(z), int(e2m1), group, _p(out))
    return out


def dequant(w_packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray | None, group: int,
            e2m1: bool = False, nvfp4: bool = False) -> np.ndarray:
    w = np.ascontiguousarray(w_packed, dtype=np.int32)
    N, K = w.shape[0], w.shape[1] * 8
    sc, fmt, z = _scales_arg(scales, zeros, nvfp4)
    out = np.empty((N, K), dtype=np.float64)
    lib().w4o_dequant(_p(w), N, K, _p(sc), fmt, _p(z), int(e2m1), group, _p(out))
    return out


def moe_route(logits: np.ndarray, top_k: int, renormalize: bool = True) -> tuple[np.ndarray, np.ndarray]:
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = lg.shape
    tw = np.empty((T, top_k), dtype=np.float32)
    ids = np.empty((T, top_k), dtype=np.int32)
    lib().w4o_moe_route(_p(lg), T, E, top_k, int(renormalize), _p(tw), _p(ids))
    return tw, ids


def moe_align(ids: np.ndarray, E: int, bm: int):
    """-> (sorted_ids (P,), expert_ids (ceil(P/bm),), ntp int, inv_pos (numel,))."""
    flat = np.ascontiguousarray(ids, dtype=np.int32).ravel()
    numel = flat.size
    P = numel + (E + 1) * (bm - 1)
    sorted_ids = np.empty((P,), dtype=np.int32)
    expert_ids = np.empty(((P + bm - 1) // bm,), dtype=np.int32)
    ntp = np.zeros((1,), dtype=np.int32)
    inv = np.empty((max(numel, 1),), dtype=np.int32)
    lib().w4o_moe_align(_p(flat), numel, E, bm, _p(sorted_ids), _p(expert_ids), _p(ntp), _p(inv))
    return sorted_ids, expert_ids, int(ntp[0]), inv[:numel]


def moe_forward(x_bits, dtype, tw, sorted_ids, expert_ids, ntp, bm, top_k, w13, s13, z13, w2, s2, z2,
                e2m1=False, with_buf2=False, nvfp4=False, round_y2=False):
    """Full grouped W4A8 MoE forward in f64 -> (T, H) (before the dtype cast). nvfp4: e4m3 block-scale
    bytes in s13/s2 and the (E, N) f32 globals in z13/z2. round_y2: each slot's gemm2 row rounded to
    the dtype before the combine (the reference's unfused gemm2 + gather-reduce); else unrounded (its
    fused gemm2 + gather-reduce)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    T, H = x.shape
    E, N1 = w13.shape[0], w13.shape[1]
    I = N1 // 2
    g1 = H // s13.shape[1]
    g2 = I // s2.shape[1]
    fmt = 2 if nvfp4 else 0 if s13.dtype == np.float16 else 1
    conv = (lambda a: np.ascontiguousarray(a).view(np.uint16)) if fmt == 0 else (lambda a: np.ascontiguousarray(a, dtype=np.uint8))
    a13, a2 = conv(s13), conv(s2)
    w13c, w2c = np.ascontiguousarray(w13, dtype=np.int32), np.ascontiguousarray(w2, dtype=np.int32)
    zc = (lambda z: np.ascontiguousarray(np.asarray(z, dtype=np.float32)).view(np.int32)) if nvfp4 else \
        (lambda z: np.ascontiguousarray(z, dtype=np.int32))
    z13c = None if z13 is None else zc(z13)
    z2c = None if z2 is None else zc(z2)
    out = np.empty((T, H), dtype=np.float64)
    buf2 = np.zeros((max(ntp, 1), I), dtype=np.uint16) if with_buf2 else None
    twc = np.ascontiguousarray(tw, dtype=np.float32)
    lib().w4o_moe_forward(_p(x), dtype, T, H, I, E, top_k, _p(twc), _p(np.ascontiguousarray(sorted_ids, dtype=np.int32)),
                          _p(np.ascontiguousarray(expert_ids, dtype=np.int32)), ntp, bm, _p(w13c), _p(a13), _p(z13c),
                          _p(w2c), _p(a2), _p(z2c), fmt, int(e2m1), g1, g2, _p(out), _p(buf2), int(round_y2))
    return (out, buf2) if with_buf2 else out


def w4a16_moe_forward(x_bits, dtype, tw, ids, w13, s13, z13, w2, s2, z2, e2m1=False, nvfp4=False):
    """Grouped W4A16 MoE forward in f64 -> ((T, H) f64 before the dtype cast, (T*top_k, I) h bits):
    x decoded exactly from its bf16 (dtype 0) / fp16 (dtype 1) bits, slots straight from the route
    ids (T, top_k). Weights and scales as in moe_forward."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    T, H = x.shape
    E, N1 = w13.shape[0], w13.shape[1]
    I = N1 // 2
    g1 = H // s13.shape[1]
    g2 = I // s2.shape[1]
    fmt = 2 if nvfp4 else 0 if s13.dtype == np.float16 else 1
    conv = (lambda a: np.ascontiguousarray(a).view(np.uint16)) if fmt == 0 else (lambda a: np.ascontiguousarray(a, dtype=np.uint8))
    zc = (lambda z: np.ascontiguousarray(np.asarray(z, dtype=np.float32)).view(np.int32)) if nvfp4 else \
        (lambda z: np.ascontiguousarray(z, dtype=np.int32))
    idc = np.ascontiguousarray(ids, dtype=np.int32)
    top_k = idc.shape[1]
    out = np.empty((T, H), dtype=np.float64)
    h = np.zeros((T * top_k, I), dtype=np.uint16)
    lib().w4o_w4a16_moe_forward(_p(x), dtype, T, H, I, E, top_k, _p(np.ascontiguousarray(tw, dtype=np.float32)),
                                _p(idc), _p(np.ascontiguousarray(w13, dtype=np.int32)), _p(conv(s13)),
                                _p(None if z13 is None else zc(z13)), _p(np.ascontiguousarray(w2, dtype=np.int32)),
                                _p(conv(s2)), _p(None if z2 is None else zc(z2)), fmt, int(e2m1), g1, g2, _p(out), _p(h))
    return out, h


def silu_mul(gate: float, up: float, dtype: int = 0) -> int:
    return int(lib().w4o_silu_mul(gate, up, dtype))


def rms_norm(x_bits: np.ndarray, weight_bits: np.ndarray | None, eps: float, dtype: int = 0, plus_one: bool = False,
             residual_bits: np.ndarray | None = None):
    """RMSNorm (+ residual add) over (M, K) bf16/fp16 bit patterns -> (out bits, new residual bits or None)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    M, K = x.shape
    out = np.empty_like(x)
    res = None if residual_bits is None else np.ascontiguousarray(residual_bits, dtype=np.uint16).copy()
    w = None if weight_bits is None else np.ascontiguousarray(weight_bits, dtype=np.uint16)
    lib().w4o_rms_norm(_p(x), _p(res), _p(w), int(plus_one), float(eps), dtype, M, K, _p(out))
    return out, res


def act_split(x_bits: np.ndarray, dtype: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """W4A16 activation split of (M, K) bf16 (dtype 0) / fp16 (dtype 1) bit patterns -> (codes (T*M, K)
    u8, scales (T*M,) f32), T = 2 for bf16, 3 for fp16."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    M, K = x.shape
    T = 2 if dtype == 0 else 3
    q = np.empty((T * M, K), dtype=np.uint8)
    s = np.empty((T * M,), dtype=np.float32)
    lib().w4o_act_split(_p(x), dtype, M, K, _p(q), _p(s))
    return q, s


def w4a16_gemm(x_bits: np.ndarray, dtype: int, w_packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray | None,
               group: int, e2m1: bool = False, nvfp4: bool = False) -> np.ndarray:
    """f64 y = x @ dequant(W)^T with x decoded exactly from its bf16/fp16 bits (the unquantized
    activations of python/minisgl/quant/kernels.py:1125-1178)."""
    xb = np.ascontiguousarray(x_bits, dtype=np.uint16)
    if dtype == 0:
        x = bf16_to_f32(xb).astype(np.float64)
    else:
        x = xb.view(np.float16).astype(np.float64)
    return x @ dequant(w_packed, scales, zeros, group, e2m1, nvfp4).T
