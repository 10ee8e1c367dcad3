"""Imports the package's host module (its directory name is not a Python identifier)."""
import importlib.util
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "granite-4-rtx-4070-ti-super_amd")
HEADER = os.path.join(ROOT, "include", "granite4_layerops.h")


def layerops():
    if "g4_layerops" in sys.modules:
        return sys.modules["g4_layerops"]
    spec = importlib.util.spec_from_file_location("g4_layerops",
                                                  os.path.join(PKG_DIR, "layerops.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["g4_layerops"] = mod
    spec.loader.exec_module(mod)
    return mod
