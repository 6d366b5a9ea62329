"""Host side of the selective scan for this package's operator layer.

The compiled module is the PyTorch-ROCm extension ``_ext/selective_scan``
(host C++ over the C ABI of libssm_mamba_hip.so), the counterpart of the
reference's ``selective_scan`` module (``csrc/selective_scan/bindings.cpp:5-8``):
its ``forward`` / ``backward`` keep the reference's argument order, validation
messages (``RuntimeError``) and padding rule (``"right"`` unless given;
``csrc/selective_scan/selective_scan.cpp:248``), and its ``h`` is the
reference's (prod a, h) chunk carry.

The ``forward`` / ``backward`` here are the extended form the operator layer
and the model harness use (``fwd_ext`` / ``bwd_ext``):

* u / delta / B / C / dout (and the optional z) may be float32 or bfloat16
  (one dtype for all of them); A, D, delta_bias, h_init are float32.
* The chunk-state carrier ``h`` holds the state after every 16 steps, shape
  (batch, ceil(seqlen/16), state_dim, dim), float32, channel-contiguous, so the
  kernels' saves and reloads are coalesced; ``h[:, -1].transpose(1, 2)`` is
  the final state.  (The reference-API ``forward`` returns the reference's
  (prod a, h) carry per 128-step chunk, (batch, dim, ceil(seqlen/128),
  2*state_dim), a view of a buffer that also holds these 16-step states.)
* Keyword extensions: ``z`` (fused output gate out * silu(z)),
  ``delta_softplus`` and, for ``forward``, ``save_chunks=False`` (inference:
  only the final state is produced).
* With z, ``forward(..., out_ungated=y)`` also writes the ungated output
  D*u + sum_n C*h into y, and ``backward`` takes it back
  (``out_ungated=y``, required with z) for dz = dy * y * silu'(z); the
  reference applies the gate outside the kernel, where autograd saves the
  same tensor.
"""
from __future__ import annotations

from typing import List, Optional

import torch

from . import _ext as _E

CHUNK = 16  # steps between saved states (SSM_CHUNK of the C ABI)


def _ext():
    return _E.module("selective_scan")


def bc_batch_strided(B: torch.Tensor, C: torch.Tensor) -> bool:
    """Whether B and C (batch, state_dim, seq_len) can be passed as they are:
    rows contiguous, the rows of a batch row seq_len apart, one batch stride
    shared by B and C (a channel slice of the x-projection output is)."""
    if B.dim() != 3 or C.dim() != 3 or B.shape != C.shape:
        return False
    batch, nstate, seqlen = B.shape
    for x in (B, C):
        if x.stride(2) != 1 or (nstate > 1 and x.stride(1) != seqlen):
            return False
        if batch > 1 and x.stride(0) < nstate * seqlen:
            return False
    return batch == 1 or B.stride(0) == C.stride(0)


def _bc_stride(B: torch.Tensor) -> int:
    """The bc_batch_stride argument (0: contiguous)."""
    batch, nstate, seqlen = B.shape
    return 0 if (batch == 1 or B.stride(0) == nstate * seqlen) else B.stride(0)


def nchunks(seqlen: int) -> int:
    return (seqlen + CHUNK - 1) // CHUNK


def last_state(h: torch.Tensor) -> torch.Tensor:
    """Final state (batch, dim, state_dim) of a chunk-state carrier, as a view."""
    return h[:, -1].transpose(1, 2)


def forward(u: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
            D: Optional[torch.Tensor], delta: torch.Tensor, delta_bias: Optional[torch.Tensor],
            h_init: Optional[torch.Tensor] = None, length: Optional[torch.Tensor] = None,
            padding_side: Optional[str] = None, *, z: Optional[torch.Tensor] = None,
            delta_softplus: bool = True, save_chunks: bool = True,
            out_ungated: Optional[torch.Tensor] = None) -> List[torch.Tensor]:
    """Returns [out, h]: out (batch, dim, seqlen) in u's dtype (gated by silu(z)
    when z is given) and h, the chunk-state carrier (batch, nchunks,
    state_dim, dim) float32 -- or, with save_chunks=False, the final state
    (batch, dim, state_dim).  out_ungated (with z): a (batch, dim, seqlen)
    tensor of u's dtype that receives the output before the gate."""
    return _ext().fwd_ext(u, A, B, C, D, delta, delta_bias, h_init, length, padding_side, z,
                          bool(delta_softplus), 1 if save_chunks else 0, out_ungated)


def backward(u: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
             D: Optional[torch.Tensor], delta: torch.Tensor, delta_bias: Optional[torch.Tensor],
             h: torch.Tensor, h_init: Optional[torch.Tensor], dout: torch.Tensor,
             dh_last: Optional[torch.Tensor], length: Optional[torch.Tensor] = None,
             padding_side: Optional[str] = None, *, z: Optional[torch.Tensor] = None,
             delta_softplus: bool = True,
             out_ungated: Optional[torch.Tensor] = None) -> List[Optional[torch.Tensor]]:
    """Returns [du, dA, dB, dC, dD, ddelta, ddelta_bias, dh_init] (+ [dz] when z
    is given), the reference's order (``selective_scan.cpp:376``).  dD /
    ddelta_bias are None when D / delta_bias are None; dh_init is None without
    h_init.  With z, out_ungated is the forward's ungated output.  h may be
    the state layout of this module's forward or the pair view of the
    extension's reference-API forward."""
    res = _ext().bwd_ext(u, A, B, C, D, delta, delta_bias, h, h_init, dout, dh_last, length,
                         padding_side, z, bool(delta_softplus), out_ungated)
    return list(res[:8]) + ([res[8]] if z is not None else [])
