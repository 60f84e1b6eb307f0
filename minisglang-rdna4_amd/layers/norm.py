"""RMSNorm producers for the W4A8 linears: the norm, the fused residual-add norm, and their fp8 form.

Mirrors python/minisgl/layers/norm.py of the reference: `_rms_norm` (:9-24), `_rms_norm_quant`
(:27-46), `_rms_norm_add_quant` (:49-58), `RMSNorm.forward` / `forward_quant` / `forward_inplace`
(:61-96) and `RMSNormFused.forward` / `forward_quant` (:125-168). All of them run one native kernel
(`w4a8_rms_norm`): the norm over the f32-widened row, rounded to the activation dtype, times the
gain in that dtype, and, for the `_quant` forms, the per-token fp8 pair of that rounded output as
an epilogue, bit for bit what `kernels.act_quant(out)` returns (uint8 e4m3 codes, f32 scales). A w4a8 linear given the pair
(`x_fp8=`, `act_scales=`) skips its own act-quant launch and re-read of the rows.

The native kernel covers bf16 and fp16 rows of up to 32768 elements. `_rms_norm_quant` and
`_rms_norm_add_quant` return None outside that (the reference's "kernel does not apply" answer,
after which the caller does not pass a pair and the linear quantizes as before); the plain norm
raises there, since this package carries no other implementation of it.
"""
from __future__ import annotations

import importlib
from typing import Tuple

import torch

_pkg = __name__.rsplit(".", 2)[0]
_abi = importlib.import_module(f"{_pkg}._abi")
engaged = importlib.import_module(f"{_pkg}._hip_engage").engaged

_MAX_K = 32768


def _native_ok(*ts: torch.Tensor | None) -> bool:
    x = ts[0]
    if x.dtype not in (torch.bfloat16, torch.float16) or not x.is_cuda or x.shape[-1] > _MAX_K or x.shape[-1] % 8:
        return False
    return all(t is None or (t.dtype == x.dtype and t.is_cuda) for t in ts[1:])


def _launch(x: torch.Tensor, weight: torch.Tensor | None, eps: float, plus_one: bool,
            residual: torch.Tensor | None, quant: bool, out: torch.Tensor | None = None):
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    M = x2.shape[0]
    o = torch.empty((M, K), dtype=x.dtype, device=x.device) if out is None else out.view(M, K)
    w = None if weight is None else weight.contiguous()
    r2 = None if residual is None else residual.view(M, K)
    xq = xs = None
    if quant:
        xq = torch.empty((M, K), dtype=torch.uint8, device=x.device)
        xs = torch.empty((M,), dtype=torch.float32, device=x.device)
    lib = _abi.load()
    _abi.check(lib.w4a8_rms_norm(_abi.ptr(x2), _abi.dtype_code(x.dtype), M, K, x2.stride(0), _abi.ptr(r2),
                                 K if r2 is None else r2.stride(0), _abi.ptr(w), int(bool(plus_one)), float(eps),
                                 _abi.ptr(o), o.stride(0), _abi.ptr(xq), K, _abi.ptr(xs), _abi.stream_of(x)),
               "rms_norm")
    o = o.view(x.shape)
    if not quant:
        return o
    return o, xq.view(x.shape), xs


def _rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float, plus_one: bool = False) -> torch.Tensor:
    """fp32-internal RMSNorm over the last dim, output in x's dtype (python/minisgl/layers/norm.py:9-24).
    weight None: the unweighted norm; plus_one: the (1 + weight) gain."""
    if not _native_ok(x, weight):
        raise TypeError(f"rms_norm: bf16/fp16 CUDA rows of at most {_MAX_K} elements (multiple of 8) only; got "
                        f"{x.dtype} {tuple(x.shape)}")
    engaged("w4a8_mi355x.rms_norm")
    return _launch(x, weight, eps, plus_one, None, False)


def _rms_norm_quant(x: torch.Tensor, weight: torch.Tensor | None, eps: float,
                    plus_one: bool = False) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None:
    """The same norm plus the fp8-e4m3 form of its own output row: (out, x_fp8, act_scales), or None
    when the native kernel does not apply (python/minisgl/layers/norm.py:27-46)."""
    if not _native_ok(x, weight):
        return None
    engaged("w4a8_mi355x.rms_norm_quant")
    return _launch(x, weight, eps, plus_one, None, True)


def _rms_norm_add_quant(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor | None, eps: float,
                        plus_one: bool = False) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None:
    """`_rms_norm_quant` for the fused residual-add norm: `residual` becomes x + residual in place (the
    SAME storage) and the norm runs over it (python/minisgl/layers/norm.py:49-58)."""
    if not _native_ok(x, residual, weight) or not residual.is_contiguous() or residual.shape != x.shape:
        return None
    engaged("w4a8_mi355x.rms_norm_add_quant")
    return _launch(x, weight, eps, plus_one, residual, True)


def _rms_norm_add(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor | None, eps: float,
                  plus_one: bool = False) -> torch.Tensor:
    if not _native_ok(x, residual, weight) or not residual.is_contiguous() or residual.shape != x.shape:
        raise TypeError("rms_norm_add: bf16/fp16 CUDA rows and a contiguous residual of the same shape only")
    engaged("w4a8_mi355x.rms_norm_add")
    return _launch(x, weight, eps, plus_one, residual, False)


class RMSNorm:
    """python/minisgl/layers/norm.py:61-96."""

    def __init__(self, size: int, eps: float, *, plus_one: bool = False) -> None:
        self.eps = eps
        self.plus_one = plus_one
        self.weight = torch.empty(size)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _rms_norm(x, self.weight, self.eps, self.plus_one)

    def forward_quant(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor | None, torch.Tensor | None]:
        """`forward` plus the fp8 pair for the w4a8 linears it feeds: (out, x_fp8, act_scales); the pair
        is None when the native kernel does not apply, and the caller then does not pass it."""
        r = _rms_norm_quant(x, self.weight, self.eps, self.plus_one)
        if r is None:
            return _rms_norm(x, self.weight, self.eps, self.plus_one), None, None
        return r[0], r[1], r[2]

    def forward_inplace(self, x: torch.Tensor) -> None:
        if not x.is_contiguous():
            x.copy_(_rms_norm(x, self.weight, self.eps, self.plus_one))
            return
        if not _native_ok(x, self.weight):
            raise TypeError(f"rms_norm: bf16/fp16 CUDA rows of at most {_MAX_K} elements only; got {x.dtype}")
        engaged("w4a8_mi355x.rms_norm")
        _launch(x, self.weight, self.eps, self.plus_one, None, False, out=x)  # each row read before written


class RMSNormFused:
    """python/minisgl/layers/norm.py:125-168: the norm with an optional fused residual add."""

    def __init__(self, size: int, eps: float, *, plus_one: bool = False) -> None:
        self.eps = eps
        self.plus_one = plus_one
        self.weight = torch.empty(size)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> Tuple[torch.Tensor, torch.Tensor]:
        if residual is None:
            return _rms_norm(x, self.weight, self.eps, self.plus_one), x
        # residual <- x + residual (new residual); out = rmsnorm(sum)
        return _rms_norm_add(x, residual, self.weight, self.eps, self.plus_one), residual

    def forward_quant(self, x: torch.Tensor, residual: torch.Tensor | None = None
                      ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor | None, torch.Tensor | None]:
        """`forward` plus the fp8 pair for a downstream w4a8 linear: (out, residual, x_fp8, act_scales).
        `out` and `residual` are bit-identical to `forward`; the pair is None when the native kernel
        does not apply."""
        if residual is None:
            r = _rms_norm_quant(x, self.weight, self.eps, self.plus_one)
            if r is None:
                return _rms_norm(x, self.weight, self.eps, self.plus_one), x, None, None
            return r[0], x, r[1], r[2]
        r = _rms_norm_add_quant(x, residual, self.weight, self.eps, self.plus_one)
        if r is None:
            out, res = self.forward(x, residual)
            return out, res, None, None
        return r[0], residual, r[1], r[2]
