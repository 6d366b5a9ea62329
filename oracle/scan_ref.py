"""CPU oracle for the selective-scan hot path (test infrastructure only).

This module is the parity checker.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it; the product path in
``ssm_mamba_amd`` never does, and fails loudly when its HIP library is missing.

It restates, in plain PyTorch CPU tensor arithmetic (float64 for checking,
float32 for the timed CPU baseline), what the reference computes:

* forward  -- ``csrc/selective_scan/forward_kernel.cu:136-243``
  (softplus with threshold 20 at :155-159, the (a, b) recurrence with
  a = exp(delta * A) at :166,192-195, padding masks at :196-205, h_init seeding
  at :208-215, y = D*u + sum_n C*h at :161,232-234);
* backward -- ``csrc/selective_scan/backward_kernel.cu:212-452``
  (reverse recurrence of the state adjoint at :345-366, dh_init = a_0*g_0 at
  :368-370, the per-position gradient terms at :372-383, softplus chain rule
  at :411-418, the dA/dD/d(delta_bias) reductions at :402-408,439-452 and the
  per-channel dB/dC accumulation at :385-400);
* single-step update -- ``csrc/selective_update/kernel.cu:39-71``;
* output gate z (the caller's ``hidden * silu(gate)``,
  ``modules/mamba.py:182,240``), fused here as an optional extension.

Padding (``length``): a padded position is an identity step of the recurrence
(a = 1, b = 0; ``forward_kernel.cu:196-205``), ``out`` is still produced at
every position, and the scan's backward treats the loss as not depending on
padded outputs (upstream gradient masked to zero there), which is the
reference's behaviour for right padding on its scalar-load path
(``backward_kernel.cu:225-246,299-303,374,389``).  Left padding uses the same
rule mirrored (the reference's left-padding backward is inconsistent, see the
design notes).  The z gate is the reference's elementwise product outside the
scan (``modules/mamba.py:181-182``), which autograd differentiates at every
position: dz = dy * out * silu'(z) with the unmasked dy, padded positions
included, while the scan itself receives the masked dy * silu(z).

The chunk-state carrier ``h_chunks`` holds the state at the end of every
``chunk``-step chunk, shape (B, D, nchunks, N); the reference stores the pair
(prod a, h) per 128-step chunk (``forward_kernel.cu:225-228``); only the state
half is used by any consumer.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

__all__ = [
    "EPS32",
    "error_bound",
    "softplus",
    "softplus_grad",
    "valid_mask",
    "scan_fwd",
    "scan_bwd",
    "update",
    "CHUNK",
]

# State checkpoint granularity of the GPU forward (steps per saved state).
CHUNK = 16


def softplus(x: torch.Tensor) -> torch.Tensor:
    """softplus with the reference's threshold: x <= 20 ? log1p(exp(x)) : x
    (``forward_kernel.cu:155-159``, ``selective_update/kernel.cu:56-57``)."""
    return torch.where(x <= 20.0, torch.log1p(torch.exp(torch.clamp(x, max=20.0))), x)


def softplus_grad(x: torch.Tensor) -> torch.Tensor:
    """d softplus / dx = x <= 20 ? sigmoid(x) : 1 (``backward_kernel.cu:411-416``)."""
    return torch.where(x <= 20.0, torch.sigmoid(x), torch.ones_like(x))


def _silu(z: torch.Tensor) -> torch.Tensor:
    return z * torch.sigmoid(z)


def _silu_grad(z: torch.Tensor) -> torch.Tensor:
    s = torch.sigmoid(z)
    return s * (1.0 + z * (1.0 - s))


def valid_mask(batch: int, seqlen: int, length: Optional[torch.Tensor],
               padding_right: bool) -> torch.Tensor:
    """(B, L) bool: right padding keeps t < len, left padding keeps
    L - len <= t < L (``forward_kernel.cu:196-205``).  ``len`` is clamped to
    [0, L]."""
    t = torch.arange(seqlen).unsqueeze(0)
    if length is None:
        return torch.ones(batch, seqlen, dtype=torch.bool)
    ln = length.to(torch.int64).cpu().clamp(0, seqlen).unsqueeze(1)
    if padding_right:
        return t < ln
    return t >= (seqlen - ln)


def _prep(u, delta, A, B, C, D, delta_bias, h_init, z, dtype, keep_graph=False):
    if keep_graph:
        cv = lambda x: None if x is None else x.to("cpu", dtype)
    else:
        cv = lambda x: None if x is None else x.detach().to("cpu", dtype)
    u, delta, A, B, C, D, delta_bias, h_init, z = map(
        cv, (u, delta, A, B, C, D, delta_bias, h_init, z))
    batch, dim, seqlen = u.shape
    if D is None:
        D = torch.zeros(dim, dtype=dtype)
    if delta_bias is None:
        delta_bias = torch.zeros(dim, dtype=dtype)
    return u, delta, A, B, C, D, delta_bias, h_init, z


def scan_fwd(u, delta, A, B, C, D=None, delta_bias=None, h_init=None,
             length=None, padding_right=True, z=None, delta_softplus=True,
             chunk: Optional[int] = CHUNK, dtype=torch.float64, keep_graph: bool = False,
             magnitude: bool = False):
    """Reference forward (differentiable by autograd when ``keep_graph``; the
    inputs are detached otherwise).  Returns a dict with

    * ``out``   (B,D,L) pre-gate output D*u + sum_n C*h,
    * ``y``     (B,D,L) out * silu(z) (== out without z),
    * ``h_last``(B,D,N) state after the last position,
    * ``h_chunks`` (B,D,nchunks,N) state at the end of each ``chunk`` steps,
    * ``prod_a`` (B,D,nchunks,N) product of the decays a_t from t = 0 to the
      end of each chunk (the first half of the reference's (prod a, h) chunk
      carry, ``forward_kernel.cu:225-228``).

    With ``magnitude`` every signed factor is replaced by its absolute value
    (the decays a = exp(delta*A) are positive and stay as they are), so each
    output becomes the sum of the absolute values of the terms that make it
    up: the scale of the rounding error of any evaluation of the same sums
    (see ``error_bound``).
    """
    u, delta, A, B, C, D, delta_bias, h_init, z = _prep(
        u, delta, A, B, C, D, delta_bias, h_init, z, dtype, keep_graph)
    batch, dim, seqlen = u.shape
    nstate = A.shape[1]
    x = delta + delta_bias[None, :, None]
    dt = softplus(x) if delta_softplus else x
    mask = valid_mask(batch, seqlen, length, padding_right)[:, None, :]
    dt = torch.where(mask, dt, torch.zeros_like(dt))
    gate = _silu(z) if z is not None else None
    if magnitude:
        u, B, C, D = u.abs(), B.abs(), C.abs(), D.abs()
        h_init = None if h_init is None else h_init.abs()
        gate = None if gate is None else gate.abs()
    dtu = (dt.abs() if magnitude else dt) * u
    dtsum = torch.zeros(batch, dim, dtype=dtype)
    prods = []
    h = torch.zeros(batch, dim, nstate, dtype=dtype) if h_init is None else h_init.clone()
    out = torch.empty(batch, dim, seqlen, dtype=dtype)
    chunks = []
    for t in range(seqlen):
        a = torch.exp(dt[:, :, t, None] * A[None])
        b = dtu[:, :, t, None] * B[:, None, :, t]
        h = a * h + b
        out[:, :, t] = torch.einsum("bdn,bn->bd", h, C[:, :, t])
        dtsum = dtsum + dt[:, :, t]
        if chunk and ((t + 1) % chunk == 0 or t == seqlen - 1):
            chunks.append(h.clone())
            prods.append(torch.exp(dtsum[:, :, None] * A[None]))
    out = out + D[None, :, None] * u
    y = out * gate if gate is not None else out
    res = {"out": out, "y": y, "h_last": h}
    if chunk:
        empty = torch.zeros(batch, dim, 0, nstate, dtype=dtype)
        res["h_chunks"] = torch.stack(chunks, dim=2) if chunks else empty
        res["prod_a"] = torch.stack(prods, dim=2) if prods else empty
    return res


def scan_bwd(u, delta, A, B, C, D=None, delta_bias=None, h_init=None,
             length=None, padding_right=True, z=None, delta_softplus=True,
             dy=None, dh_last=None, seg: int = 64, dtype=torch.float64,
             magnitude: bool = False):
    """Reference backward by an explicit reverse loop with state checkpoints
    every ``seg`` steps (memory O(B*D*N*(L/seg + seg))).

    Returns a dict with du, ddelta, dA, dB, dC, dD, ddelta_bias, dh_init
    (None without h_init) and dz (None without z).  ``magnitude``: as for
    ``scan_fwd``, each result becomes the sum of the absolute values of its
    terms (A enters the dA / ddelta terms by its absolute value, the decays
    exp(delta*A) unchanged).
    """
    u, delta, A, B, C, D, delta_bias, h_init, z = _prep(
        u, delta, A, B, C, D, delta_bias, h_init, z, dtype)
    dy = dy.detach().to("cpu", dtype)
    batch, dim, seqlen = u.shape
    nstate = A.shape[1]
    dh_last = (torch.zeros(batch, dim, nstate, dtype=dtype) if dh_last is None
               else dh_last.detach().to("cpu", dtype))

    x = delta + delta_bias[None, :, None]
    dt_raw = softplus(x) if delta_softplus else x
    dsp = softplus_grad(x) if delta_softplus else torch.ones_like(x)
    mask = valid_mask(batch, seqlen, length, padding_right)[:, None, :]
    dt = torch.where(mask, dt_raw, torch.zeros_like(dt_raw))
    gate = _silu(z) if z is not None else None
    gate_grad = _silu_grad(z) if z is not None else None
    Aterm = A
    if magnitude:
        u, B, C, D, dy, dh_last = u.abs(), B.abs(), C.abs(), D.abs(), dy.abs(), dh_last.abs()
        h_init = None if h_init is None else h_init.abs()
        gate = None if gate is None else gate.abs()
        if z is not None:  # silu'(z) = s (1 + z (1 - s)) by the sizes of its terms
            sz = torch.sigmoid(z)
            gate_grad = sz * (1.0 + z.abs() * (1.0 - sz))
        Aterm = A.abs()
        dsp = dsp.abs()
    dtf = dt.abs() if magnitude else dt  # the step size as a factor (decays keep dt)
    dtu = dtf * u
    dy_gate = dy  # the gate sees every position: dz = dy * out * silu'(z)
    dy = torch.where(mask, dy, torch.zeros_like(dy))
    dout = dy * gate if z is not None else dy

    # forward checkpoints: state before each segment
    h = torch.zeros(batch, dim, nstate, dtype=dtype) if h_init is None else h_init.clone()
    ckpt = []
    for s0 in range(0, seqlen, seg):
        ckpt.append(h.clone())
        for t in range(s0, min(s0 + seg, seqlen)):
            h = torch.exp(dt[:, :, t, None] * A[None]) * h + dtu[:, :, t, None] * B[:, None, :, t]

    du = torch.empty_like(u)
    dd = torch.empty_like(u)
    out_pre = torch.empty_like(u)
    dA = torch.zeros_like(A)
    dB = torch.zeros_like(B)
    dC = torch.zeros_like(C)
    gam = dh_last.clone()          # d loss / d h_t from the future (times a_{t+1})
    for si in reversed(range(len(ckpt))):
        s0 = si * seg
        s1 = min(s0 + seg, seqlen)
        hs = [ckpt[si]]
        for t in range(s0, s1):
            hs.append(torch.exp(dt[:, :, t, None] * A[None]) * hs[-1]
                      + dtu[:, :, t, None] * B[:, None, :, t])
        for t in reversed(range(s0, s1)):
            a = torch.exp(dt[:, :, t, None] * A[None])
            h_prev = hs[t - s0]
            h_t = hs[t - s0 + 1]
            Bt = B[:, None, :, t]
            Ct = C[:, None, :, t]
            out_pre[:, :, t] = torch.einsum("bdn,bdn->bd", h_t, Ct.expand_as(h_t))
            G = gam + dout[:, :, t, None] * Ct
            gB = (G * Bt).sum(-1)
            gah = G * a * h_prev
            du[:, :, t] = D[None, :] * dout[:, :, t] + dtf[:, :, t] * gB
            dd[:, :, t] = u[:, :, t] * gB + (gah * Aterm[None]).sum(-1)
            dA += (gah * dtf[:, :, t, None]).sum(0)
            dB[:, :, t] = (G * dtu[:, :, t, None]).sum(1)
            dC[:, :, t] = (dout[:, :, t, None] * h_t).sum(1)
            gam = a * G
    ddelta = torch.where(mask, dd * dsp, torch.zeros_like(dd))
    res = {
        "du": du,
        "ddelta": ddelta,
        "dA": dA,
        "dB": dB,
        "dC": dC,
        "dD": (dout * u).sum((0, 2)),
        "ddelta_bias": ddelta.sum((0, 2)),
        "dh_init": gam if h_init is not None else None,
        "dz": None,
    }
    if z is not None:
        out_pre = out_pre + D[None, :, None] * u
        res["dz"] = dy_gate * out_pre * gate_grad
    return res


def update(state, x, dt, A, B, C, D=None, dt_bias=None, z=None,
           dt_softplus=True, dtype=torch.float64, magnitude: bool = False):
    """Single decode step (``selective_update/kernel.cu:39-71``):
    delta = softplus(dt + bias); h' = exp(delta*A)*h + delta*x*B;
    out = D*x + sum_n C*h' (then * silu(z) when z is given).  Returns
    (out, new_state); ``state`` is not modified.  ``magnitude``: as for
    ``scan_fwd`` (sums of the absolute values of the terms)."""
    cv = lambda t: None if t is None else t.detach().to("cpu", dtype)
    state, x, dt, A, B, C, D, dt_bias, z = map(cv, (state, x, dt, A, B, C, D, dt_bias, z))
    batch, dim = x.shape
    if D is None:
        D = torch.zeros(dim, dtype=dtype)
    if dt_bias is None:
        dt_bias = torch.zeros(dim, dtype=dtype)
    v = dt + dt_bias[None, :]
    delta = softplus(v) if dt_softplus else v
    a = torch.exp(delta[:, :, None] * A[None])
    gate = _silu(z) if z is not None else None
    if magnitude:
        state, x, B, C, D, delta = state.abs(), x.abs(), B.abs(), C.abs(), D.abs(), delta.abs()
        gate = None if gate is None else gate.abs()
    new = a * state + (delta * x)[:, :, None] * B[:, None, :]
    out = torch.einsum("bdn,bn->bd", new, C) + D[None, :] * x
    if gate is not None:
        out = out * gate
    return out, new


# Unit roundoff of float32 (round to nearest).
EPS32 = 2.0 ** -24


def error_bound(ref: torch.Tensor, mag: Optional[torch.Tensor], rtol: float, atol: float,
                c: float, eps: float = EPS32) -> torch.Tensor:
    """Per-element tolerance for a float32 evaluation of a result whose
    float64 value is ``ref`` and whose terms have absolute values summing to
    ``mag`` (the ``magnitude`` mode of this module):
    atol + rtol * |ref| + c * EPS32 * mag.  The last term is the classical
    bound on the rounding error of a sum (or recurrence) of terms evaluated in
    float32, (number of roundings along the longest chain) * u * sum |terms|
    (Higham, "Accuracy and Stability of Numerical Algorithms", 2nd ed., §4.2),
    with c standing for that chain length; it matters only where the terms
    cancel, so that |ref| is small against their sizes.  ``eps`` is the unit
    roundoff of the arithmetic being bounded (2^-8 where the values pass
    through bfloat16 between operations)."""
    r = ref.detach().double().cpu()
    b = atol + rtol * r.abs()
    if mag is not None:
        b = b + c * eps * mag.detach().double().cpu()
    return b


def algorithmic_bytes_scan(batch, dim, seqlen, nstate, s_in, s_bc, has_z):
    """Unique HBM bytes of one forward and one backward call (each tensor read or
    written once): returns (fwd_bytes, bwd_bytes)."""
    s_z = s_in if has_z else 0
    fwd = (batch * dim * seqlen * (3 * s_in + s_z)         # u, delta, out (+z)
           + batch * nstate * seqlen * 2 * s_bc             # B, C
           + dim * nstate * 4 + 2 * dim * 4                 # A, D, bias
           + batch * dim * nstate * 4)                      # last state
    bwd = (batch * dim * seqlen * (5 * s_in + 2 * s_z)      # u, delta, dout, du, ddelta (+z, dz)
           + batch * nstate * seqlen * 4 * s_bc             # B, C, dB, dC
           + 2 * dim * nstate * 4 + 4 * dim * 4             # A, dA, D, bias, dD, dbias
           + batch * dim * nstate * 4)                      # dlast
    return fwd, bwd


def algorithmic_bytes_update(batch, dim, nstate, s_in, s_bc, has_z):
    s_z = s_in if has_z else 0
    return (2 * batch * dim * nstate * 4 + batch * dim * (3 * s_in + s_z)
            + dim * nstate * 4 + 2 * dim * 4 + batch * nstate * 2 * s_bc)


def inv_softplus(x: torch.Tensor) -> torch.Tensor:
    """dt + log(-expm1(-dt)): the inverse of softplus used to initialise
    delta_bias (``modules/mamba.py:62-69``)."""
    return x + torch.log(-torch.expm1(-x))


def make_inputs(batch, dim, seqlen, nstate, seed=0, dtype=torch.float32,
                with_z=True, delta_shift=0.0, h_init=False):
    """Synthetic inputs with the reference's init distributions: u, z, delta ~
    N(0,1); A = -(1..N) broadcast over channels (S4D-real,
    ``modules/mamba.py:71-73,166``); delta_bias = inv_softplus of log-uniform dt
    in [1e-3, 0.1] clamped at 1e-4 (``modules/mamba.py:62-69``); B, C ~ N(0,1);
    D = 1 (``modules/mamba.py:75``).  Values are generated in float32 on the CPU
    and rounded once to ``dtype`` for u/delta/z/B/C."""
    g = torch.Generator().manual_seed(seed)
    f32 = torch.float32
    u = torch.randn(batch, dim, seqlen, generator=g, dtype=f32)
    delta = torch.randn(batch, dim, seqlen, generator=g, dtype=f32) + delta_shift
    z = torch.randn(batch, dim, seqlen, generator=g, dtype=f32) if with_z else None
    Bm = torch.randn(batch, nstate, seqlen, generator=g, dtype=f32)
    Cm = torch.randn(batch, nstate, seqlen, generator=g, dtype=f32)
    A = -torch.arange(1, nstate + 1, dtype=f32)[None, :].expand(dim, nstate).contiguous()
    dtv = torch.exp(torch.rand(dim, generator=g, dtype=f32) * (math.log(0.1) - math.log(1e-3))
                    + math.log(1e-3)).clamp(min=1e-4)
    bias = inv_softplus(dtv)
    Dv = torch.ones(dim, dtype=f32)
    hi = torch.randn(batch, dim, nstate, generator=g, dtype=f32) if h_init else None
    rd = lambda t: None if t is None else t.to(dtype)
    return {
        "u": rd(u), "delta": rd(delta), "A": A, "B": rd(Bm), "C": rd(Cm),
        "D": Dv, "delta_bias": bias, "z": rd(z), "h_init": hi,
    }
