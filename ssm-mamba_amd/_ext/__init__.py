"""The PyTorch-ROCm extension modules of this package, built in-tree by
``_build.py``:

* ``selective_scan``   -- ``forward`` / ``backward`` with the reference's
  argument order (``csrc/selective_scan/bindings.cpp:5-8``), plus the
  extended ``fwd_ext`` / ``bwd_ext``;
* ``selective_update`` -- ``apply`` (``csrc/selective_update/bindings.cpp:5-7``)
  plus ``apply_ext``.

Both are host C++ over the C ABI of ``_lib/libssm_mamba_hip.so``.  With this
directory on ``sys.path`` they import under the reference's top-level names
(``import selective_scan``), which is how the reference's ``ops/`` files find
them.  There is no fallback: a missing module raises.
"""
from __future__ import annotations

import importlib

import torch  # noqa: F401  -- the modules link against libtorch / libc10_hip

_mods = {}


def module(name: str):
    """The built extension module ``name`` (selective_scan or selective_update)."""
    m = _mods.get(name)
    if m is None:
        try:
            m = importlib.import_module(f"{__name__}.{name}")
        except ImportError as e:
            raise RuntimeError(
                f"ssm_mamba_amd: extension module {name} is not built ({e}); build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'`") from e
        _mods[name] = m
    return m
