"""Host side of the decode step: the counterpart of the reference's compiled
``selective_update`` module (``csrc/selective_update/bindings.cpp:5-7``) and
its ``apply`` entry point, over the C ABI of libssm_mamba_hip.so.

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

from . import _native as N
from .selective_scan import _STREAM_DTYPES, _check, _check_dim, _ptr, _stream


def _validate(u, A, B, C, D, delta, delta_bias, h, z):
    _check_dim(u, 2, "u")
    _check_dim(A, 2, "A")
    _check_dim(B, 2, "B")
    _check_dim(C, 2, "C")
    if D is not None:
        _check_dim(D, 1, "D")
    _check_dim(delta, 2, "delta")
    if delta_bias is not None:
        _check_dim(delta_bias, 1, "delta_bias")
    _check_dim(h, 3, "h")
    batch, dim, nstate = h.shape
    if nstate > 256:
        raise RuntimeError("selective_update only supports state_dim <= 256")
    sd = (torch.float32, torch.bfloat16)
    f32 = (torch.float32,)
    _check(u, "u", (batch, dim), "batch_size, num_channels", sd, "float32 or bfloat16")
    io = (u.dtype,)
    io_txt = str(u.dtype).replace("torch.", "") + " (the dtype of u)"
    _check(A, "A", (dim, nstate), "num_channels, state_dim", f32, "float32")
    _check(B, "B", (batch, nstate), "batch_size, state_dim", io, io_txt)
    _check(C, "C", (batch, nstate), "batch_size, state_dim", io, io_txt)
    if D is not None:
        _check(D, "D", (dim,), "num_channels", f32, "float32")
    _check(delta, "delta", (batch, dim), "batch_size, num_channels", io, io_txt)
    if delta_bias is not None:
        _check(delta_bias, "delta_bias", (dim,), "num_channels", f32, "float32")
    _check(h, "h", (batch, dim, nstate), "batch_size, num_channels, state_dim", f32, "float32")
    if z is not None:
        _check(z, "z", (batch, dim), "batch_size, num_channels", io, io_txt)
    return batch, dim, nstate


def apply_ext(u: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
              D: Optional[torch.Tensor], delta: torch.Tensor, delta_bias: Optional[torch.Tensor],
              h: torch.Tensor, *, z: Optional[torch.Tensor] = None, delta_softplus: bool = True,
              inplace: bool = False, out: Optional[torch.Tensor] = None) -> List[torch.Tensor]:
    """One decode step; returns [out, new_h].  With inplace=True, new_h is h
    (updated in place)."""
    batch, dim, nstate = _validate(u, A, B, C, D, delta, delta_bias, h, z)
    L = N.lib()
    dev = u.device
    if out is None:
        out = torch.empty_like(u)
    new_h = h if inplace else torch.empty_like(h)
    with torch.cuda.device(dev):
        N.check(L.ssm_selective_state_update(
            batch, dim, nstate, _STREAM_DTYPES[u.dtype], h.data_ptr(), new_h.data_ptr(),
            u.data_ptr(), delta.data_ptr(), A.data_ptr(), B.data_ptr(), C.data_ptr(), _ptr(D),
            _ptr(delta_bias), _ptr(z), 1 if delta_softplus else 0, out.data_ptr(), _stream(dev)))
    return [out, new_h]


def apply(u: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, D: torch.Tensor,
          delta: torch.Tensor, delta_bias: torch.Tensor, h: torch.Tensor) -> List[torch.Tensor]:
    """Reference-compatible step: returns [out, new_h], h is not modified."""
    return apply_ext(u, A, B, C, D, delta, delta_bias, h)
