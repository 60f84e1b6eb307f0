"""MI355X-native (gfx950 / CDNA4) W4A8 quantized-linear path of minisglang-rdna4.

Mirrors the reference's provider API (``minisgl.quant.kernels`` / ``minisgl.quant.method`` /
``minisgl.quant.mxfp4`` and the MoE quant methods of ``minisgl.layers.moe``) on top of
hand-written HIP kernels reached through the C ABI in ``include/w4a8_mi355x.h``.

The directory name is not a Python identifier, so import it with importlib::

    pkg = importlib.import_module("minisglang-rdna4_amd")
    kernels = importlib.import_module("minisglang-rdna4_amd.quant.kernels")
"""
from __future__ import annotations

__version__ = "0.1.0"

from . import _abi  # noqa: F401
