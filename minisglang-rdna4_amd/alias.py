"""Register this package's modules under the reference's module names (the drop-in at the Python API).

The reference's engine imports its quantized-linear provider as ``minisgl.quant.kernels`` and its
method layer as ``minisgl.quant.method`` / ``minisgl.quant.config`` / ``minisgl.quant.mxfp4`` /
``minisgl.quant.nvfp4`` and ``minisgl.layers.moe`` / ``minisgl.layers.norm``. This package's directory
name is not a Python identifier, so it cannot be imported under those names directly; ``install()``
puts the modules into ``sys.modules`` under them. Names the reference defines and this package does
not (its engine, models, other quant schemes) are not created: importing them still fails.
"""
from __future__ import annotations

import importlib
import sys
import types

_pkg = __name__.rsplit(".", 1)[0]

_MODULES = {
    "quant.kernels": "quant.kernels",
    "quant.method": "quant.method",
    "quant.config": "quant.config",
    "quant.mxfp4": "quant.mxfp4",
    "quant.nvfp4": "quant.nvfp4",
    "quant.loader": "quant.loader",
    "layers.moe": "layers.moe",
    "layers.norm": "layers.norm",
}


def install(prefix: str = "minisgl", *, replace: bool = False) -> dict[str, types.ModuleType]:
    """Make ``{prefix}.quant.kernels`` etc. resolve to this package's modules. Existing entries are
    left alone unless ``replace`` (an engine that already imported its own ``minisgl.quant`` keeps it).
    Returns the modules registered, by name."""
    done: dict[str, types.ModuleType] = {}

    def put(name: str, mod: types.ModuleType) -> None:
        if replace or name not in sys.modules:
            sys.modules[name] = mod
            done[name] = mod

    def parent(name: str) -> types.ModuleType:
        mod = sys.modules.get(name)
        if mod is None:
            mod = types.ModuleType(name)
            mod.__path__ = []  # a package, so submodule imports resolve through sys.modules
            put(name, mod)
        return mod

    root = parent(prefix)
    for sub in ("quant", "layers"):
        setattr(root, sub, parent(f"{prefix}.{sub}"))
    for alias, real in _MODULES.items():
        mod = importlib.import_module(f"{_pkg}.{real}")
        name = f"{prefix}.{alias}"
        put(name, mod)
        head, leaf = name.rsplit(".", 1)
        setattr(sys.modules[head], leaf, sys.modules[name])
    return done
