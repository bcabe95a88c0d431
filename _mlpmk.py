"""Registers the package directory ``mlp-megakernel_amd/`` (whose name is not a
Python identifier) under the import name ``mlpmk``.

``import _mlpmk`` once; afterwards ``import mlpmk`` / ``from mlpmk import ops``
work anywhere in the process.
"""
import importlib.util
import os
import sys

PKG_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mlp-megakernel_amd")


def _load():
    mod = sys.modules.get("mlpmk")
    if mod is not None:
        return mod
    spec = importlib.util.spec_from_file_location(
        "mlpmk", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR]
    )
    mod = importlib.util.module_from_spec(spec)
    sys.modules["mlpmk"] = mod
    try:
        spec.loader.exec_module(mod)
    except BaseException:
        sys.modules.pop("mlpmk", None)
        raise
    return mod


mlpmk = _load()
