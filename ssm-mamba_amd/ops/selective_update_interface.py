"""Drop-in replacement of ``ops/selective_update_interface.py`` of the reference.

``SelectiveUpdateFn.apply`` keeps the reference's signature and out-of-place
contract (``ops/selective_update_interface.py:8-44``).  ``selective_state_update``
is the functional decode step: it returns the output and updates ``state`` in
place.
"""
from __future__ import annotations

from typing import Optional

import torch

from .. import selective_update
from ..utils.tensor_utils import ensure_contiguous


class SelectiveUpdateFn:
    @staticmethod
    def apply(u: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
              D: torch.Tensor, delta: torch.Tensor, delta_bias: torch.Tensor, h: torch.Tensor):
        """
        u, delta: (batch, channels); A: (channels, state_dim); B, C: (batch, state_dim);
        D, delta_bias: (channels,); h: (batch, channels, state_dim).
        Returns out (batch, channels) and the new state (batch, channels, state_dim).
        """
        u = ensure_contiguous(u)
        A = ensure_contiguous(A.float())
        B = ensure_contiguous(B.to(u.dtype))
        C = ensure_contiguous(C.to(u.dtype))
        D = ensure_contiguous(D.float())
        delta = ensure_contiguous(delta.to(u.dtype))
        delta_bias = ensure_contiguous(delta_bias.float())
        h = ensure_contiguous(h.float())
        out, h = selective_update.apply(u, A, B, C, D, delta, delta_bias, h)
        return out, h


def selective_state_update(state: torch.Tensor, x: torch.Tensor, dt: torch.Tensor,
                           A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                           D: Optional[torch.Tensor] = None, z: Optional[torch.Tensor] = None,
                           dt_bias: Optional[torch.Tensor] = None,
                           dt_softplus: bool = True) -> torch.Tensor:
    """One decode step.  state (batch, channels, state_dim) float32 is updated
    in place; returns out (batch, channels) in x's dtype."""
    if state.dtype != torch.float32 or not state.is_contiguous():
        raise RuntimeError("state must be a contiguous float32 tensor (it is updated in place)")
    io = x.dtype
    x = ensure_contiguous(x)
    dt = ensure_contiguous(dt.to(io))
    B = ensure_contiguous(B.to(io))
    C = ensure_contiguous(C.to(io))
    z = None if z is None else ensure_contiguous(z.to(io))
    A = ensure_contiguous(A.float())
    D = None if D is None else ensure_contiguous(D.float())
    dt_bias = None if dt_bias is None else ensure_contiguous(dt_bias.float())
    out, _ = selective_update.apply_ext(x, A, B, C, D, dt, dt_bias, state, z=z,
                                        delta_softplus=dt_softplus, inplace=True)
    return out
