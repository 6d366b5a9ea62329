"""Drop-in replacement of ``ops/selective_scan_interface.py`` of the reference.

``SelectiveScanFn`` keeps the reference's positional signature
(``ops/selective_scan_interface.py:9-21``), contiguity handling (:40-43), the
saved tensors (:52-58), the (out, h_last) return (:60) and the 10-gradient
backward (:62-80).  ``selective_scan_fn`` is the functional form with the
optional fused gate z, optional D / delta_bias, the softplus switch and
``return_last_state``.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import selective_scan
from ..utils.tensor_utils import ensure_contiguous


def _fp32(x: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return x if x is None or x.dtype == torch.float32 else x.float()


def _as(x: Optional[torch.Tensor], dtype) -> Optional[torch.Tensor]:
    return x if x is None or x.dtype == dtype else x.to(dtype)


class SelectiveScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, u: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                D: torch.Tensor, delta: torch.Tensor, delta_bias: torch.Tensor,
                h_init: Optional[torch.Tensor] = None, length: Optional[torch.Tensor] = None,
                padding_size: str = "left") -> Tuple[torch.Tensor, torch.Tensor]:
        """
        u, delta: (batch, channels, seq_len); A: (channels, state_dim);
        B, C: (batch, state_dim, seq_len); D, delta_bias: (channels,);
        h_init: (batch, channels, state_dim); length: (batch,) int64.
        Returns out (batch, channels, seq_len) and h_last (batch, channels, state_dim).
        """
        u, A, B, C, D, delta, delta_bias, h_init, length = map(
            ensure_contiguous, (u, A, B, C, D, delta, delta_bias, h_init, length))
        io = u.dtype
        A32, D32, bias32, h0 = _fp32(A), _fp32(D), _fp32(delta_bias), _fp32(h_init)
        B, C, delta = _as(B, io), _as(C, io), _as(delta, io)
        need_grad = any(ctx.needs_input_grad)
        out, h = selective_scan.forward(u, A32, B, C, D32, delta, bias32, h0, length,
                                        padding_size, save_chunks=need_grad)
        if need_grad:
            ctx.save_for_backward(u, A32, B, C, D32, delta, bias32, h, h0, length)
            ctx.padding_size = padding_size
            return out, selective_scan.last_state(h)
        return out, h

    @staticmethod
    def backward(ctx, dout, dh_last):
        if not hasattr(ctx, "saved_tensors") or len(ctx.saved_tensors) == 0:
            return (None,) * 10
        u, A, B, C, D, delta, delta_bias, h, h_init, length = ctx.saved_tensors
        dout = ensure_contiguous(dout.to(u.dtype))
        dh_last = None if dh_last is None else ensure_contiguous(dh_last.float())
        du, dA, dB, dC, dD, ddelta, ddelta_bias, dh_init = selective_scan.backward(
            u, A, B, C, D, delta, delta_bias, h, h_init, dout, dh_last, length, ctx.padding_size)
        return du, dA, dB, dC, dD, ddelta, ddelta_bias, dh_init, None, None


class _SelectiveScanExtFn(torch.autograd.Function):
    """Autograd wrapper of the extended forward/backward (z gate, optional D /
    delta_bias, softplus switch)."""

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D, z, delta_bias, h_init, length, delta_softplus,
                padding_side):
        io = u.dtype
        u, delta, z = (ensure_contiguous(_as(t, io)) for t in (u, delta, z))
        B, C = _as(B, io), _as(C, io)
        # batch-strided B / C views (a slice of the x-projection output) go to
        # the kernels as they are; other layouts are made contiguous
        if not selective_scan.bc_batch_strided(B, C):
            B, C = ensure_contiguous(B), ensure_contiguous(C)
        A32, D32, bias32, h0 = (ensure_contiguous(_as(t, torch.float32))
                                for t in (A, D, delta_bias, h_init))
        length = ensure_contiguous(length)
        need_grad = any(ctx.needs_input_grad)
        # with the gate, the backward needs the ungated output (what autograd
        # saves for the reference's out * silu(z) outside the kernel)
        y = torch.empty_like(u) if (need_grad and z is not None) else None
        out, h = selective_scan.forward(u, A32, B, C, D32, delta, bias32, h0, length, padding_side,
                                        z=z, delta_softplus=delta_softplus, save_chunks=need_grad,
                                        out_ungated=y)
        if need_grad:
            ctx.save_for_backward(u, delta, A32, B, C, D32, z, y, bias32, h, h0, length)
            ctx.delta_softplus = delta_softplus
            ctx.padding_side = padding_side
            return out, selective_scan.last_state(h)
        return out, h

    @staticmethod
    def backward(ctx, dout, dh_last):
        u, delta, A, B, C, D, z, y, bias, h, h0, length = ctx.saved_tensors
        dout = ensure_contiguous(dout.to(u.dtype))
        dh_last = None if dh_last is None else ensure_contiguous(dh_last.float())
        res = selective_scan.backward(u, A, B, C, D, delta, bias, h, h0, dout, dh_last, length,
                                      ctx.padding_side, z=z, delta_softplus=ctx.delta_softplus,
                                      out_ungated=y)
        du, dA, dB, dC, dD, ddelta, dbias, dh0 = res[:8]
        dz = res[8] if z is not None else None
        return du, ddelta, dA, dB, dC, dD, dz, dbias, dh0, None, None, None


def selective_scan_fn(u: torch.Tensor, delta: torch.Tensor, A: torch.Tensor, B: torch.Tensor,
                      C: torch.Tensor, D: Optional[torch.Tensor] = None,
                      z: Optional[torch.Tensor] = None, delta_bias: Optional[torch.Tensor] = None,
                      delta_softplus: bool = True, return_last_state: bool = False,
                      h_init: Optional[torch.Tensor] = None, length: Optional[torch.Tensor] = None,
                      padding_side: str = "left"):
    """Functional selective scan: out = (D*u + sum_n C*h) * silu(z), returned
    alone or with the last state (batch, channels, state_dim)."""
    out, last = _SelectiveScanExtFn.apply(u, delta, A, B, C, D, z, delta_bias, h_init, length,
                                          delta_softplus, padding_side)
    return (out, last) if return_last_state else out
