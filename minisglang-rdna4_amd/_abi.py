"""ctypes binding of libw4a8_mi355x.so (declarations: include/w4a8_mi355x.h and the measurement probe
of include/w4a8_probe.h).

The library is the only compute path: if it is missing, or no GPU is present, calls raise. There
is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

_PKG = Path(__file__).resolve().parent
_LIB_PATH = _PKG / "_lib" / "libw4a8_mi355x.so"

BF16, F16, F32 = 0, 1, 2
SCALE_F16, SCALE_E8M0, SCALE_E4M3 = 0, 1, 2
W_INT4, W_E2M1 = 0, 1
# status codes (w4a8_mi355x.h)
ERR_UNSUPPORTED = 2
KERNEL_AUTO, KERNEL_DECODE, KERNEL_PREFILL = 0, 1, 2

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_vp = ctypes.c_void_p

# name -> (restype, argtypes); must match include/w4a8_mi355x.h
SIGNATURES = {
    "w4a8_abi_version": (_c_int, []),
    "w4a8_last_error": (ctypes.c_char_p, []),
    "w4a8_act_quant": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp, _vp]),
    "w4a8_tile_bytes": (_c_i64, [_c_i64, _c_i64]),
    "w4a8_repack_weights": (_c_int, [_vp, _c_i64, _c_i64, _c_int, _vp, _vp]),
    "w4a8_gemm_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_int]),
    "w4a8_gemm": (_c_int, [_vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_int, _vp, _c_int, _c_i64,
                           _vp, _c_int, _c_i64, _c_int, _vp, _c_i64, _c_int, _vp]),
    "w4a8_linear_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "w4a8_linear": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _vp, _c_int, _vp, _c_int, _c_i64,
                             _vp, _c_int, _c_i64, _c_int, _vp, _c_i64, _c_int, _vp]),
    # measurement probe (include/w4a8_probe.h), not part of the W4A8 path
    "w4a8_probe_read": (_c_int, [_vp, _c_i64, _c_int, _c_int, _c_int, _vp, _vp]),
    "w4a8_linear_launch_count": (_c_int, [_c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_int,
                                          _c_int]),
    "w4a8_linear_noalloc_max_bytes": (_c_i64, []),
    "w4a8_linear_noalloc": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _vp, _c_int, _vp, _c_int,
                                     _c_i64, _vp, _c_int, _c_i64, _c_int, _c_int, _vp]),
    "w4a8_moe_route": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_int, _c_int, _vp, _vp, _vp]),
    "w4a8_rms_norm": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _vp, _c_int, ctypes.c_float, _vp,
                               _c_i64, _vp, _c_i64, _vp, _vp]),
    "w4a8_moe_route_align": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_i64, _vp, _vp, _vp,
                                      _vp, _vp, _vp, _vp, _c_int, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp]),
    "w4a8_moe_route_slots": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_i64, _vp, _vp, _vp,
                                      _vp, _vp, _vp, _vp, _c_int, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp]),
    "w4a8_moe_padded_capacity": (_c_i64, [_c_i64, _c_i64, _c_int]),
    "w4a8_moe_align": (_c_int, [_vp, _c_i64, _c_i64, _c_int, _c_i64, _vp, _vp, _vp, _vp, _vp]),
    "w4a8_moe_gemm_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_int, _c_i64, _c_i64, _c_i64, _c_int]),
    "w4a8_moe_gemm": (_c_int, [_vp, _c_i64, _vp, _c_int, _vp, _vp, _vp, _c_i64, _c_int, _c_int, _c_i64,
                               _vp, _c_i64, _c_i64, _c_i64, _vp, _c_int, _vp, _c_int, _c_i64,
                               _vp, _c_int, _c_i64, _c_int, _vp, _c_i64, _c_int, _vp]),
    "w4a8_moe_gemm_quant_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "w4a8_moe_gemm_quant": (_c_int, [_vp, _c_int, _c_i64, _vp, _vp, _vp, _c_i64, _c_int, _c_i64, _vp, _c_i64, _c_i64,
                                     _c_i64, _vp, _c_int, _vp, _c_int, _c_i64, _vp, _c_int, _c_i64, _vp, _c_i64,
                                     _c_int, _vp]),
    "w4a8_moe_combine": (_c_int, [_vp, _c_int, _c_i64, _vp, _vp, _c_i64, _c_int, _c_i64, _vp, _c_int, _vp]),
    "w4a8_moe_gelu_tanh_mul": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp]),
    "w4a8_moe_gemm2_combine_supported": (_c_int, [_c_i64, _c_int, _c_int, _c_int, _c_i64, _c_int]),
    "w4a8_moe_gemm2_combine": (_c_int, [_vp, _c_int, _c_i64, _vp, _vp, _vp, _c_i64, _c_int, _c_int, _c_i64, _vp,
                                        _c_i64, _c_i64, _c_i64, _vp, _c_int, _vp, _c_int, _c_i64, _vp, _c_int,
                                        _c_i64, _c_int, _vp]),
    "w4a8_moe_route_gemm1": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_int, _c_int, _vp, _c_int, _c_i64, _c_int,
                                      _c_i64, _vp, _c_i64, _c_i64, _vp, _c_int, _vp, _c_int, _c_i64, _vp, _vp, _vp,
                                      _vp, _vp, _vp, _vp, _c_int, _c_i64, _vp]),
    "w4a16_act_split": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp]),
    "w4a16_linear_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_int]),
    "w4a16_linear": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _vp, _c_int, _vp, _c_int, _c_i64,
                              _vp, _c_i64, _c_int, _vp, _c_i64, _c_int, _vp]),
    "w4a16_moe_silu_split": (_c_int, [_vp, _c_i64, _vp, _c_i64, _c_int, _c_i64, _c_int, _vp, _c_i64, _vp, _vp,
                                      _c_i64, _vp]),
}

_lock = threading.Lock()
_lib = None


def lib_path() -> Path:
    return Path(os.environ.get("W4A8_MI355X_LIB", str(_LIB_PATH)))


def load() -> ctypes.CDLL:
    """Load the shared library (once) and bind every declared symbol."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        if not path.exists():
            raise RuntimeError(
                f"libw4a8_mi355x.so not built ({path}); run __graft_entry__.build() or "
                f"python minisglang-rdna4_amd/build.py"
            )
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().w4a8_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg or f'status {rc}'}")


def ptr(t) -> int | None:
    """Device pointer of a torch tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


def stream_of(t) -> int:
    import torch

    return torch.cuda.current_stream(t.device).cuda_stream


def dtype_code(dt) -> int:
    import torch

    if dt == torch.bfloat16:
        return BF16
    if dt == torch.float16:
        return F16
    if dt == torch.float32:
        return F32
    raise TypeError(f"unsupported dtype {dt}")
