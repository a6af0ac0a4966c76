"""MI355X-native (gfx950) implementation of the Seera GEMM / Conv2D /
ConvTranspose2D hot path.

* ``libseera_hip.so`` -- hand-written HIP kernels behind the C ABI of
  ``include/seera_hip.h``; driven from Python through :mod:`.capi` (ctypes).
* ``seera_cuda`` -- pybind11 module with the reference's function names and
  signatures (engine_cuda/src/cuda_bindings.cpp), so the reference's
  ``cuTen.py`` / ``Seera_Engine.py`` can ``import seera_cuda`` unchanged.

Build in-tree with ``python -m ml_framework_amd.build``.
"""
from __future__ import annotations

import importlib
import os
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))


def seera_cuda():
    """Import the compiled ``seera_cuda`` module (raises if not built)."""
    mod = importlib.import_module("ml_framework_amd.seera_cuda")
    # Importing the submodule binds it to this package's attribute of the same
    # name; put the loader back so that later calls keep working.
    globals()["seera_cuda"] = _load_seera_cuda
    return mod


_load_seera_cuda = seera_cuda


def install_seera_cuda() -> None:
    """Make ``import seera_cuda`` resolve to this package's module, as the
    reference's cuTen.py:3 expects."""
    sys.modules.setdefault("seera_cuda", seera_cuda())
