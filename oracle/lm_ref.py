"""CPU oracle of the Mamba causal-LM glue around the scan (test infrastructure
only: imported by ``tests/`` and never by the product package).

It restates, token-major and in float64 by default, what the reference's
modules compute, reading parameters from a ``state_dict`` with the reference's
names:

* ``rms_norm``      -- ``modules/rms_norm.py:11-31``: x*rsqrt(mean x^2 + eps)*(1+w);
* ``causal_conv``   -- the depthwise ``nn.Conv1d`` with padding k-1, first L
  outputs kept (``modules/mamba.py:37-44,138``), as an explicit tap loop;
* ``mamba_forward`` -- ``modules/mamba.py:82-187``: in-projection split into
  (x, gate), conv + SiLU, x-projection split into (delta_r, B, C), delta =
  W_dt @ delta_r with the bias handed to the scan, A = -exp(log_A), the scan
  with ``lengths`` and the reference call's default left padding (under
  autograd the scan's gradient is dropped at padded outputs, as the
  reference's backward kernel does), the gate out*silu(gate), out-projection; with use_cache, the conv window of the k-1
  pre-conv inputs ending at lengths-1 (zero before the sequence start,
  :113-135) and the last state;
* ``mamba_step``    -- ``modules/mamba.py:189-243``;
* the residual block inside ``lm_forward`` / ``lm_step`` --
  ``modules/block.py:50-87`` (eval mode: dropout is the identity);
* ``lm_forward`` / ``lm_step`` / ``generate`` -- ``models/causal_lm.py:75-133``.

The scan and the single-step update are ``oracle.scan_ref.scan_fwd`` /
``update``.  ``lm_forward`` keeps the autograd graph (parameters that require
grad get float64 gradients of the exact forward), which is the check for a
training step.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import torch

from .scan_ref import scan_fwd, update, valid_mask

__all__ = ["rms_norm", "causal_conv", "mamba_forward", "mamba_step", "lm_forward", "lm_step",
           "generate", "layer_params"]


def _silu(x: torch.Tensor) -> torch.Tensor:
    return x / (1.0 + torch.exp(-x))


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Normalise over the last axis (``modules/rms_norm.py:11-31``)."""
    return x * torch.rsqrt((x * x).mean(dim=-1, keepdim=True) + eps) * (1.0 + weight)


def causal_conv(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor]) -> torch.Tensor:
    """Depthwise causal conv over x (batch, channels, L) with weight
    (channels, 1, k): out[t] = sum_j w[j] * x[t - (k-1) + j], x = 0 before t=0."""
    batch, ch, seqlen = x.shape
    k = weight.shape[-1]
    out = torch.zeros_like(x)
    for j in range(k):
        shift = k - 1 - j
        if shift >= seqlen:
            continue
        out[:, :, shift:] += weight[None, :, 0, j, None] * x[:, :, :seqlen - shift]
    if bias is not None:
        out = out + bias[None, :, None]
    return out


def layer_params(sd: Dict[str, torch.Tensor], i: int, dtype=torch.float64) -> Dict[str, torch.Tensor]:
    """The parameters of layer i from a CausalLM state_dict, as ``dtype`` on the CPU."""
    pre = f"layers.{i}."
    return {k[len(pre):]: v.to("cpu", dtype) for k, v in sd.items() if k.startswith(pre)}


def mamba_forward(p: Dict[str, torch.Tensor], x: torch.Tensor, state_dim: int, delta_rank: int,
                  h0: Optional[torch.Tensor] = None, lengths: Optional[torch.Tensor] = None,
                  use_cache: bool = False, prefix: str = "ssm.", state_mag: Optional[list] = None):
    """x (batch, L, model_dim) -> (y (batch, L, model_dim), last state
    (batch, inner, N), conv window (batch, inner, k-1) or None).  With a list
    ``state_mag``, the scan's magnitude run (sums of |terms| of the last
    state, ``scan_fwd(..., magnitude=True)``) is appended to it."""
    g = lambda n: p.get(prefix + n)
    batch, seqlen, _ = x.shape
    w_in = g("input_proj.weight")
    inner = w_in.shape[0] // 2
    xz = x @ w_in.t()
    if g("input_proj.bias") is not None:
        xz = xz + g("input_proj.bias")
    xs = xz[..., :inner].permute(0, 2, 1)              # (batch, inner, L)
    gate = xz[..., inner:].permute(0, 2, 1)
    conv_w = g("conv.weight")
    k = conv_w.shape[-1]
    ctx = None
    if use_cache:
        lens = torch.full((batch,), seqlen, dtype=torch.long) if lengths is None else lengths.cpu()
        ctx = torch.zeros(batch, inner, k - 1, dtype=x.dtype)
        for b in range(batch):
            for j in range(k - 1):
                t = int(lens[b]) - (k - 1) + j
                if t >= 0:
                    ctx[b, :, j] = xs[b, :, t]
    xc = _silu(causal_conv(xs, conv_w, g("conv.bias")))
    params = xc.permute(0, 2, 1) @ g("ssm_param_proj.weight").t()   # (batch, L, R + 2N)
    dr = params[..., :delta_rank]
    Bm = params[..., delta_rank:delta_rank + state_dim].permute(0, 2, 1)
    Cm = params[..., delta_rank + state_dim:].permute(0, 2, 1)
    delta = (dr @ g("delta_proj.weight").t()).permute(0, 2, 1)
    A = -torch.exp(g("log_A"))
    res = scan_fwd(xc, delta, A, Bm, Cm, g("D"), g("delta_proj.bias"), h0,
                   None if lengths is None else lengths.cpu(), padding_right=False, z=gate,
                   chunk=None, dtype=x.dtype, keep_graph=True)
    out = res["out"]
    if lengths is not None:
        # the scan's backward drops the gradient of its padded outputs
        # (backward_kernel.cu:241-246; the reference call's left padding),
        # while the gate outside it (modules/mamba.py:181-182) is
        # differentiated at every position: same values, that gradient rule
        m = valid_mask(batch, seqlen, lengths.cpu(), False)[:, None, :].to(out.dtype)
        out = out * m + (out * (1.0 - m)).detach()
    y_gated = out * _silu(gate)
    if state_mag is not None:
        sm = scan_fwd(xc, delta, A, Bm, Cm, g("D"), g("delta_proj.bias"), h0,
                      None if lengths is None else lengths.cpu(), padding_right=False, z=gate,
                      chunk=None, dtype=x.dtype, magnitude=True)["h_last"]
        # the conv window holds in-projection outputs: their terms' sizes
        wm = None
        if ctx is not None:
            xm = (x.abs() @ w_in[:inner].abs().t()).permute(0, 2, 1)
            if g("input_proj.bias") is not None:
                xm = xm + g("input_proj.bias")[:inner].abs()[None, :, None]
            wm = torch.zeros_like(ctx)
            for b in range(batch):
                for j in range(k - 1):
                    t = int(lens[b]) - (k - 1) + j
                    if t >= 0:
                        wm[b, :, j] = xm[b, :, t]
        state_mag.append((sm, wm))
    y = y_gated.permute(0, 2, 1) @ g("out_proj.weight").t()
    if g("out_proj.bias") is not None:
        y = y + g("out_proj.bias")
    return y, res["h_last"], ctx


def mamba_step(p: Dict[str, torch.Tensor], x: torch.Tensor, ctx: torch.Tensor, state: torch.Tensor,
               state_dim: int, delta_rank: int, prefix: str = "ssm."):
    """x (batch, model_dim) -> (y (batch, model_dim), new window, new state)."""
    g = lambda n: p.get(prefix + n)
    w_in = g("input_proj.weight")
    inner = w_in.shape[0] // 2
    xz = x @ w_in.t()
    if g("input_proj.bias") is not None:
        xz = xz + g("input_proj.bias")
    xs, gate = xz[:, :inner], xz[:, inner:]
    window = torch.cat([ctx, xs[..., None]], dim=-1)
    xc = (window * g("conv.weight")[:, 0, :]).sum(dim=-1)
    if g("conv.bias") is not None:
        xc = xc + g("conv.bias")
    xc = _silu(xc)
    params = xc @ g("ssm_param_proj.weight").t()
    dr = params[:, :delta_rank]
    Bv = params[:, delta_rank:delta_rank + state_dim]
    Cv = params[:, delta_rank + state_dim:]
    delta = dr @ g("delta_proj.weight").t()
    A = -torch.exp(g("log_A"))
    out, new_state = update(state, xc, delta, A, Bv, Cv, g("D"), g("delta_proj.bias"), z=gate,
                            dtype=x.dtype)
    y = out @ g("out_proj.weight").t()
    if g("out_proj.bias") is not None:
        y = y + g("out_proj.bias")
    return y, window[..., 1:].clone(), new_state


def _dims(sd: Dict[str, torch.Tensor]) -> Tuple[int, int, int]:
    n_layers = 1 + max(int(k.split(".")[1]) for k in sd if k.startswith("layers."))
    state_dim = sd["layers.0.ssm.log_A"].shape[1]
    delta_rank = sd["layers.0.ssm.delta_proj.weight"].shape[1]
    return n_layers, state_dim, delta_rank


def lm_forward(sd: Dict[str, torch.Tensor], input_ids: torch.Tensor,
               lengths: Optional[torch.Tensor] = None, use_cache: bool = False,
               dtype=torch.float64, logits_at: Optional[torch.Tensor] = None,
               extras: Optional[dict] = None):
    """logits (batch, L, vocab) and, with use_cache, the per-layer caches
    [(window, state)] (``models/causal_lm.py:75-91``).

    logits_at (batch, P) int64: only the logits at those positions,
    (batch, P, vocab) -- the LM head at every position of a long prompt is
    most of the work.  extras (a dict): receives "hidden", the normalized
    final hidden state at those positions (the LM head's input), and
    "state_mag", per layer (the magnitude run of the scan's last state, the
    sizes of the conv window's in-projection terms or None)."""
    n_layers, state_dim, delta_rank = _dims(sd)
    cv = lambda t: t.to("cpu", dtype)
    x = cv(sd["embedding.weight"])[input_ids.cpu()]
    caches: List[Tuple[torch.Tensor, torch.Tensor]] = []
    mags = [] if extras is not None else None
    for i in range(n_layers):
        p = layer_params(sd, i, dtype)
        h = rms_norm(x, p["norm.weight"])
        y, last, ctx = mamba_forward(p, h, state_dim, delta_rank, lengths=lengths,
                                     use_cache=use_cache, state_mag=mags)
        x = x + y
        caches.append((ctx, last))
    if logits_at is not None:
        x = torch.gather(x, 1, logits_at.cpu()[:, :, None].expand(-1, -1, x.shape[-1]))
    x = rms_norm(x, cv(sd["norm.weight"]))
    if extras is not None:
        extras["hidden"] = x
        extras["state_mag"] = mags
    return x @ cv(sd["lm_head.weight"]).t(), caches


def lm_step(sd: Dict[str, torch.Tensor], input_ids: torch.Tensor, caches, dtype=torch.float64,
            extras: Optional[dict] = None):
    """logits (batch, vocab) for one token and the advanced caches
    (``models/causal_lm.py:93-104``); extras (a dict) receives "hidden", the
    LM head's input."""
    n_layers, state_dim, delta_rank = _dims(sd)
    cv = lambda t: t.detach().to("cpu", dtype)
    x = cv(sd["embedding.weight"])[input_ids.cpu()]
    new = []
    for i in range(n_layers):
        p = layer_params(sd, i, dtype)
        ctx, state = caches[i]
        y, ctx, state = mamba_step(p, rms_norm(x, p["norm.weight"]), ctx, state, state_dim,
                                   delta_rank)
        x = x + y
        new.append((ctx, state))
    x = rms_norm(x, cv(sd["norm.weight"]))
    if extras is not None:
        extras["hidden"] = x
    return x @ cv(sd["lm_head.weight"]).t(), new


def generate(sd: Dict[str, torch.Tensor], input_ids: torch.Tensor, max_new_tokens: int,
             temperature: float = 1.0, pad_id: int = 0, eos_id: int = 2, dtype=torch.float64):
    """The reference's greedy loop (``models/causal_lm.py:106-133``)."""
    ids = input_ids.cpu()
    batch = ids.shape[0]
    lengths = (ids != pad_id).sum(dim=1)
    logits, caches = lm_forward(sd, ids, lengths, use_cache=True, dtype=dtype)
    logits = logits[torch.arange(batch), lengths - 1]
    seq = ids
    finished = torch.zeros(batch, dtype=torch.bool)
    for _ in range(max_new_tokens):
        if temperature != 1.0:
            logits = logits / temperature
        nxt = torch.softmax(logits, dim=-1).argmax(dim=-1, keepdim=True)
        seq = torch.cat([seq, nxt], dim=1)
        finished |= nxt[:, 0] == eos_id
        if bool(finished.all()):
            break
        logits, caches = lm_step(sd, nxt[:, 0], caches, dtype=dtype)
    after = (seq == eos_id).to(torch.int32).cumsum(dim=1) >= 1
    return torch.where(after, torch.full_like(seq, eos_id), seq)
