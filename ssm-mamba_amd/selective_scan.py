"""Host side of the selective scan: the counterpart of the reference's compiled
``selective_scan`` module (``csrc/selective_scan/bindings.cpp:5-8``) with its
``forward`` and ``backward`` entry points, implemented over the C ABI of
libssm_mamba_hip.so.

Argument order, shapes, the validation messages (``RuntimeError``) and the
``padding_side`` rule (``"right"`` unless given otherwise;
``csrc/selective_scan/selective_scan.cpp:248``) follow the reference.
Differences, all deliberate:

* u / delta / B / C / dout (and the optional z) may be float32 or bfloat16
  (one dtype for all of them); A, D, delta_bias, h_init are float32.
* The chunk-state carrier ``h`` returned by ``forward`` and consumed by
  ``backward`` holds the state after every 16 steps, shape
  (batch, ceil(seqlen/16), state_dim, dim), float32, channel-contiguous so
  the kernels' saves and reloads are coalesced; ``h[:, -1].transpose(1, 2)``
  is the final state (the reference stores (prod a, h) pairs per 128 steps,
  ``(batch, dim, nchunks, 2*state_dim)``, and takes ``h[..., -1, 1::2]``).
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

from . import _native as N

_STREAM_DTYPES = {torch.float32: N.SSM_F32, torch.bfloat16: N.SSM_BF16}


def _check_dim(x: torch.Tensor, n: int, name: str) -> None:
    if x.dim() != n:
        raise RuntimeError(f"{name} must be a {n}D tensor")


def _check(x: torch.Tensor, name: str, shape, shape_txt: str, dtypes, dtype_txt: str,
           contiguous: bool = True) -> None:
    if not x.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if x.dtype not in dtypes:
        raise RuntimeError(f"{name} must be {dtype_txt} tensor")
    if contiguous and not x.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if tuple(x.shape) != tuple(shape):
        raise RuntimeError(f"{name} must have shape ({shape_txt})")


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


def _ptr(x: Optional[torch.Tensor]):
    return None if x is None else x.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _validate(u, A, B, C, D, delta, delta_bias, h_init, length, z):
    _check_dim(u, 3, "u")
    _check_dim(A, 2, "A")
    _check_dim(B, 3, "B")
    _check_dim(C, 3, "C")
    if D is not None:
        _check_dim(D, 1, "D")
    _check_dim(delta, 3, "delta")
    if delta_bias is not None:
        _check_dim(delta_bias, 1, "delta_bias")
    if h_init is not None:
        _check_dim(h_init, 3, "h_init")
    if length is not None:
        _check_dim(length, 1, "length")
    batch, dim, seqlen = u.shape
    nstate = A.shape[1]
    if nstate > 256:
        raise RuntimeError("selective_scan only supports state_dim <= 256")
    sd = (torch.float32, torch.bfloat16)
    f32 = (torch.float32,)
    _check(u, "u", (batch, dim, seqlen), "batch_size, num_channels, seq_len", sd, "float32 or bfloat16")
    io = (u.dtype,)
    io_txt = str(u.dtype).replace("torch.", "") + " (the dtype of u)"
    _check(A, "A", (dim, nstate), "num_channels, state_dim", f32, "float32")
    # B and C may also be batch-strided views (bc_batch_strided)
    bc_ok = bc_batch_strided(B, C)
    _check(B, "B", (batch, nstate, seqlen), "batch_size, state_dim, seq_len", io,
           io_txt, contiguous=not bc_ok)
    _check(C, "C", (batch, nstate, seqlen), "batch_size, state_dim, seq_len", io, io_txt,
           contiguous=not bc_ok)
    if D is not None:
        _check(D, "D", (dim,), "num_channels", f32, "float32")
    _check(delta, "delta", (batch, dim, seqlen), "batch_size, num_channels, seq_len", io, io_txt)
    if delta_bias is not None:
        _check(delta_bias, "delta_bias", (dim,), "num_channels", f32, "float32")
    if h_init is not None:
        _check(h_init, "h_init", (batch, dim, nstate), "batch_size, num_channels, state_dim", f32, "float32")
    if z is not None:
        _check(z, "z", (batch, dim, seqlen), "batch_size, num_channels, seq_len", io, io_txt)
    if length is not None:
        if not length.is_cuda:
            raise RuntimeError("length must be a CUDA tensor")
        if length.dtype != torch.int64:
            raise RuntimeError("length must be long tensor")
        if not length.is_contiguous():
            raise RuntimeError("length must be contiguous")
        if length.shape[0] != batch:
            raise RuntimeError("length must have shape (batch_size,)")
    return batch, dim, seqlen, nstate


def nchunks(seqlen: int) -> int:
    return (seqlen + N.SSM_CHUNK - 1) // N.SSM_CHUNK


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
    batch, dim, seqlen, nstate = _validate(u, A, B, C, D, delta, delta_bias, h_init, length, z)
    if out_ungated is not None:
        if z is None:
            raise RuntimeError("out_ungated requires z")
        _check(out_ungated, "out_ungated", (batch, dim, seqlen), "batch_size, num_channels, seq_len",
               (u.dtype,), str(u.dtype).replace("torch.", "") + " (the dtype of u)")
    L = N.lib()
    dev = u.device
    out = torch.empty_like(u)
    if save_chunks:
        h = torch.empty(batch, nchunks(seqlen), nstate, dim, device=dev, dtype=torch.float32)
        h_chunks, h_last = h, None
    else:
        h = torch.empty(batch, dim, nstate, device=dev, dtype=torch.float32)
        h_chunks, h_last = None, h
    wsb = L.ssm_scan_fwd_workspace_bytes(batch, dim, seqlen, nstate)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    padding_right = 1 if (padding_side or "right") == "right" else 0
    with torch.cuda.device(dev):
        N.check(L.ssm_selective_scan_fwd(
            batch, dim, seqlen, nstate, _STREAM_DTYPES[u.dtype],
            u.data_ptr(), delta.data_ptr(), A.data_ptr(), B.data_ptr(), C.data_ptr(),
            _bc_stride(B), _ptr(D), _ptr(delta_bias), _ptr(h_init), _ptr(length), padding_right,
            _ptr(z), 1 if delta_softplus else 0, out.data_ptr(), _ptr(out_ungated), _ptr(h_chunks),
            _ptr(h_last), ws.data_ptr(), wsb, _stream(dev)))
    return [out, h]


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
    h_init.  With z, out_ungated is the forward's ungated output."""
    batch, dim, seqlen, nstate = _validate(u, A, B, C, D, delta, delta_bias, h_init, length, z)
    if (z is None) != (out_ungated is None):
        raise RuntimeError("backward with z requires out_ungated (the forward's ungated output)"
                           if z is not None else "out_ungated requires z")
    if out_ungated is not None:
        _check(out_ungated, "out_ungated", (batch, dim, seqlen), "batch_size, num_channels, seq_len",
               (u.dtype,), str(u.dtype).replace("torch.", "") + " (the dtype of u)")
    _check_dim(h, 4, "h")
    _check(h, "h", (batch, nchunks(seqlen), nstate, dim),
           "batch_size, num_chunks, state_dim, num_channels", (torch.float32,), "float32")
    _check_dim(dout, 3, "dout")
    _check(dout, "dout", (batch, dim, seqlen), "batch_size, num_channels, seq_len", (u.dtype,),
           str(u.dtype).replace("torch.", "") + " (the dtype of u)")
    if dh_last is not None:
        _check(dh_last, "dh_last", (batch, dim, nstate), "batch_size, num_channels, state_dim",
               (torch.float32,), "float32")
    L = N.lib()
    dev = u.device
    du = torch.empty_like(u)
    ddelta = torch.empty_like(delta)
    dA = torch.empty_like(A)
    dB = torch.empty_like(B)
    dC = torch.empty_like(C)
    dD = torch.empty_like(D) if D is not None else None
    dbias = torch.empty_like(delta_bias) if delta_bias is not None else None
    dh_init = torch.empty_like(h_init) if h_init is not None else None
    dz = torch.empty_like(z) if z is not None else None
    wsb = L.ssm_scan_bwd_workspace_bytes(batch, dim, seqlen, nstate)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    padding_right = 1 if (padding_side or "right") == "right" else 0
    with torch.cuda.device(dev):
        N.check(L.ssm_selective_scan_bwd(
            batch, dim, seqlen, nstate, _STREAM_DTYPES[u.dtype],
            u.data_ptr(), delta.data_ptr(), A.data_ptr(), B.data_ptr(), C.data_ptr(),
            _bc_stride(B), _ptr(D), _ptr(delta_bias), _ptr(h_init), _ptr(length), padding_right,
            _ptr(z), _ptr(out_ungated), 1 if delta_softplus else 0, h.data_ptr(), dout.data_ptr(),
            _ptr(dh_last),
            du.data_ptr(), ddelta.data_ptr(), dA.data_ptr(), dB.data_ptr(), dC.data_ptr(),
            _ptr(dD), _ptr(dbias), _ptr(dh_init), _ptr(dz), ws.data_ptr(), wsb, _stream(dev)))
    res = [du, dA, dB, dC, dD, ddelta, dbias, dh_init]
    if z is not None:
        res.append(dz)
    return res
