"""Causal depthwise conv1d (+ SiLU) over channel-major activations, on the HIP
kernels of libssm_mamba_hip.so (``ssm_causal_conv1d_fwd`` / ``_bwd``).

It computes what the reference's Mamba layer does with two torch ops,
``F.silu(self.conv(x)[..., :seq_len])`` with ``self.conv`` a depthwise
``nn.Conv1d(padding=k-1)`` (``modules/mamba.py:37-44,138-139``), as one
memory-bound pass over x (batch, channels, seq_len).  The backward writes dx
and the weight / bias gradients (deterministic fixed-order sums).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native as N

_DTYPES = {torch.float32: N.SSM_F32, torch.bfloat16: N.SSM_BF16}


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _check_x(x: torch.Tensor) -> None:
    if x.dim() != 3:
        raise RuntimeError("x must be a 3D tensor (batch, channels, seq_len)")
    if not x.is_cuda:
        raise RuntimeError("x must be a CUDA tensor")
    if x.dtype not in _DTYPES:
        raise RuntimeError("x must be float32 or bfloat16 tensor")


class CausalConv1dFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                silu: bool, lengths: Optional[torch.Tensor] = None,
                window: Optional[torch.Tensor] = None) -> torch.Tensor:
        _check_x(x)
        batch, dim, seqlen = x.shape
        # a channel slice of a larger activation (each batch row's (channels,
        # seq_len) block contiguous) is read in place through its batch stride
        if not (x.stride(2) == 1 and x.stride(1) == seqlen
                and (batch == 1 or x.stride(0) >= dim * seqlen)):
            x = x.contiguous()
        xbs = 0 if batch == 1 else x.stride(0)
        width = weight.shape[-1]
        if weight.numel() != dim * width:
            raise RuntimeError("weight must have shape (channels, 1, width) or (channels, width)")
        w = weight.reshape(dim, width).to(x.dtype).contiguous()
        b = None if bias is None else bias.to(x.dtype).contiguous()
        if b is not None and b.numel() != dim:
            raise RuntimeError("bias must have shape (channels,)")
        out = torch.empty((batch, dim, seqlen), dtype=x.dtype, device=x.device)
        if window is not None:
            if (tuple(window.shape) != (batch, dim, width - 1) or window.dtype != x.dtype
                    or not window.is_contiguous() or window.device != x.device):
                raise RuntimeError("window must be a contiguous (batch, channels, width - 1) "
                                   "tensor of x's dtype on x's device")
        if lengths is not None:
            if window is None:
                raise RuntimeError("lengths requires window")
            if (lengths.dtype != torch.int64 or tuple(lengths.shape) != (batch,)
                    or lengths.device != x.device):
                raise RuntimeError("lengths must be an int64 (batch,) tensor on x's device")
            lengths = lengths.contiguous()
        L = N.lib()
        with torch.cuda.device(x.device):
            N.check(L.ssm_causal_conv1d_fwd(batch, dim, seqlen, width, _DTYPES[x.dtype],
                                            x.data_ptr(), xbs, w.data_ptr(),
                                            None if b is None else b.data_ptr(), int(silu),
                                            out.data_ptr(),
                                            None if lengths is None else lengths.data_ptr(),
                                            None if window is None else window.data_ptr(),
                                            _stream(x.device)))
        ctx.save_for_backward(x, w, b)
        ctx.silu = silu
        ctx.weight_shape = weight.shape
        ctx.weight_dtype = weight.dtype
        ctx.bias_dtype = None if bias is None else bias.dtype
        return out

    @staticmethod
    def backward(ctx, dout: torch.Tensor):
        x, w, b = ctx.saved_tensors
        x = x.contiguous()
        batch, dim, seqlen = x.shape
        width = w.shape[1]
        dout = dout.to(x.dtype).contiguous()
        dx = torch.empty_like(x)
        dw = torch.empty_like(w)
        db = None if b is None else torch.empty_like(b)
        L = N.lib()
        nbytes = L.ssm_causal_conv1d_bwd_workspace_bytes(batch, dim, width)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        with torch.cuda.device(x.device):
            N.check(L.ssm_causal_conv1d_bwd(batch, dim, seqlen, width, _DTYPES[x.dtype],
                                            x.data_ptr(), w.data_ptr(),
                                            None if b is None else b.data_ptr(), dout.data_ptr(),
                                            int(ctx.silu), dx.data_ptr(), dw.data_ptr(),
                                            None if db is None else db.data_ptr(), ws.data_ptr(),
                                            nbytes, _stream(x.device)))
        dw = dw.reshape(ctx.weight_shape).to(ctx.weight_dtype)
        if db is not None:
            db = db.to(ctx.bias_dtype)
        return dx, dw, db, None, None, None


def causal_conv1d_fn(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                     activation: Optional[str] = "silu", *,
                     window: Optional[torch.Tensor] = None,
                     lengths: Optional[torch.Tensor] = None) -> torch.Tensor:
    """act(causal depthwise conv1d(x)) for x (batch, channels, seq_len) with
    weight (channels, 1, width) or (channels, width), width <= 8, optional bias
    (channels,); ``activation`` is "silu" or None.  ``window`` (batch,
    channels, width - 1), if given, receives the decode cache of a prefill:
    the width - 1 inputs ending at position lengths[b] - 1 (seq_len - 1
    without lengths), zero before the row start (``modules/mamba.py:113-135``)."""
    if activation not in (None, "silu"):
        raise RuntimeError("activation must be 'silu' or None")
    return CausalConv1dFn.apply(x, weight, bias, activation == "silu", lengths, window)
