"""Loader of the compiled ``_xtile`` module (``csrc/XTModule.cpp``).

The compiled module and the ctypes binding in ``_xtile.py`` present the same
functions over the same C ABI; the facade uses the ctypes binding unless
``XTILE_AMD_BINDING=compiled`` is set when the package is imported.  The
module is the counterpart of the reference's nanobind ``_xtile``
(python/XTModule.cpp:210-231), which the reference facade finds by name
(xtile/__init__.py:45-71); copying the built file into such a package as
``xtile/_xtile<ext>.so`` is how a maintainer plugs it in.
"""

from __future__ import annotations

import importlib.util
import sys
import sysconfig
from pathlib import Path

MODULE_PATH = Path(__file__).resolve().parent / "lib" / ("_xtile" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))
MODULE_NAME = "xtile_amd.lib._xtile"


def load():
    """Import the compiled module; ImportError when it is not built."""
    if MODULE_NAME in sys.modules:
        return sys.modules[MODULE_NAME]
    if not MODULE_PATH.exists():
        raise ImportError(f"{MODULE_PATH} is not built; run `python xtile_amd/build.py` (or __graft_entry__.build())")
    # torch first: its HIP runtime is the one the library's NEEDED entries
    # must bind to (one runtime per process)
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    spec = importlib.util.spec_from_file_location(MODULE_NAME, MODULE_PATH)
    module = importlib.util.module_from_spec(spec)
    sys.modules[MODULE_NAME] = module
    try:
        spec.loader.exec_module(module)
    except BaseException:
        del sys.modules[MODULE_NAME]
        raise
    return module
