"""Loads the C++ host engine (_trs_native) built in-tree next to libtrs_hip.so.

There is no CPU fallback: importing torch_rs fails loudly when the native
libraries have not been built (python pytorch-rs_amd/build.py).
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

_LIB = Path(__file__).resolve().parent.parent / "lib"


def _load():
    matches = sorted(_LIB.glob("_trs_native*.so"))
    if not matches:
        raise ImportError(f"_trs_native is not built under {_LIB}; run `python pytorch-rs_amd/build.py`")
    spec = importlib.util.spec_from_file_location("_trs_native", matches[0])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["_trs_native"] = mod
    spec.loader.exec_module(mod)
    return mod


native = sys.modules.get("_trs_native") or _load()
