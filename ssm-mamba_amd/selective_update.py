"""Host side of the decode step for this package's operator layer, over the
PyTorch-ROCm extension ``_ext/selective_update`` (host C++ over the C ABI of
libssm_mamba_hip.so), the counterpart of the reference's compiled
``selective_update`` module (``csrc/selective_update/bindings.cpp:5-7``).

``apply`` keeps the reference's argument order, its out-of-place contract
(a new state tensor is returned, ``selective_update.cpp:112-113``) and its
validation messages, and adds the device check the reference lacks.  u / delta
/ B / C may be float32 or bfloat16 (one dtype); A, D, delta_bias and the state
are float32.  ``apply_ext`` adds the fused z gate, the softplus switch and an
in-place mode.
"""
from __future__ import annotations

from typing import List, Optional

import torch

from . import _ext as _E


def _ext():
    return _E.module("selective_update")


def apply_ext(u: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
              D: Optional[torch.Tensor], delta: torch.Tensor, delta_bias: Optional[torch.Tensor],
              h: torch.Tensor, *, z: Optional[torch.Tensor] = None, delta_softplus: bool = True,
              inplace: bool = False, out: Optional[torch.Tensor] = None) -> List[torch.Tensor]:
    """One decode step; returns [out, new_h].  With inplace=True, new_h is h
    (updated in place)."""
    return _ext().apply_ext(u, A, B, C, D, delta, delta_bias, h, z, bool(delta_softplus),
                            bool(inplace), out)


def apply(u: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, D: torch.Tensor,
          delta: torch.Tensor, delta_bias: torch.Tensor, h: torch.Tensor) -> List[torch.Tensor]:
    """Reference-compatible step: returns [out, new_h], h is not modified."""
    return _ext().apply(u, A, B, C, D, delta, delta_bias, h)
