"""Shared helpers for the parity tests (HIP path vs the CPU oracle)."""
from __future__ import annotations

import os
import re
from typing import Callable, Optional, Union

import torch

from oracle import scan_ref as R

# Tolerances stated by the task for this path: fp32 rtol 1e-4 / atol 1e-5;
# bf16 inputs with fp32 accumulation rtol 2e-2 / atol 5e-3 (outputs and grads).
TOL = {
    torch.float32: dict(rtol=1e-4, atol=1e-5),
    torch.bfloat16: dict(rtol=2e-2, atol=5e-3),
}

# Rounding-chain length c of the error term c * EPS32 * sum|terms| (see
# oracle.scan_ref.error_bound).  The longest chains of float32 roundings in
# the kernels are the channel reductions of dB / dC (a 6-level DPP tree over
# 64 lanes, then up to 32 channel-block partials added in order: 38) and the
# state recurrences (one fma per step, decays < 1, so the error of a term
# from k steps back is damped by the same decay as the term).  64 covers
# both; the CPU float32 oracle needs at most 29 on the same cases.
C_CHAIN = 64

# (test, tensor, max abs err, worst err/bound, magnitude term used)
MARGINS: list = []

Mag = Optional[Union[torch.Tensor, Callable[[], torch.Tensor]]]


# Unit roundoff of bfloat16: the model harness stores its activations in the
# model dtype between operations, so a model-level result in bf16 carries
# rounding errors of this size on each term of its last operation.
EPS_BF16 = 2.0 ** -8


def assert_close(got: torch.Tensor, ref: torch.Tensor, dtype, name: str, mag: Mag = None,
                 tol: Optional[dict] = None, c: float = None, eps: float = R.EPS32):
    """Compare a GPU result with the float64 oracle at the stated tolerance,
    err <= atol + rtol * |ref| element-wise.  ``mag`` (a tensor, or a callable
    that computes it, evaluated only when needed) is the oracle's sum of the
    absolute values of each element's terms: where the plain bound fails, the
    element may also use c * EPS32 * mag, the float32 rounding error a sum of
    those terms can carry (oracle.scan_ref.error_bound).  The worst ratio of
    error to bound is recorded for the session summary."""
    t = dict(TOL[dtype] if tol is None else tol)
    c = C_CHAIN if c is None else c
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    if g.shape != r.shape:
        raise AssertionError(f"{name}: shape {tuple(g.shape)} != reference {tuple(r.shape)}")
    err = (g - r).abs()
    bound = t["atol"] + t["rtol"] * r.abs()
    used = False
    if bool((err > bound).any()) and mag is not None:
        m = mag() if callable(mag) else mag
        bound = R.error_bound(r, m, t["rtol"], t["atol"], c, eps)
        used = True
    ratio = err / bound
    worst = float(ratio.max()) if ratio.numel() else 0.0
    emax = float(err.max()) if err.numel() else 0.0
    test = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    MARGINS.append((test, name, emax, worst, used))
    if not worst <= 1.0:  # also catches NaN
        bad = ~(err <= bound)
        i = int(torch.argmax(torch.nan_to_num(ratio, nan=float("inf")).flatten()))
        raise AssertionError(
            f"{name}: {int(bad.sum())}/{err.numel()} elements out of tolerance {t}"
            f"{' + %g*%g*sum|terms|' % (c, eps) if used else ''}; worst at flat index {i}: "
            f"got {g.flatten()[i].item():.8g} ref {r.flatten()[i].item():.8g}; "
            f"max abs err {emax:.3g}, worst err/bound {worst:.3g}")


def margin_summary() -> str:
    """One line per tensor name: the worst err/bound over all checks, the
    largest absolute error, and how many checks needed the magnitude term."""
    agg = {}
    for test, name, emax, worst, used in MARGINS:
        # one line per kind of tensor: drop step / layer numbers and subsets
        key = re.sub(r"( step)? \d+$", "", name.split("[")[0])
        a = agg.setdefault(key, [0, 0.0, 0.0, "", 0])
        a[0] += 1
        a[1] = max(a[1], emax)
        if worst >= a[2]:
            a[2], a[3] = worst, test
        a[4] += int(used)
    lines = [f"{'tensor':16s} {'checks':>6s} {'max abs err':>12s} {'worst err/bound':>16s} "
             f"{'mag used':>8s}  worst in"]
    for k in sorted(agg):
        n, emax, worst, test, used = agg[k]
        lines.append(f"{k:16s} {n:6d} {emax:12.3g} {worst:16.3f} {used:8d}  {test}")
    return "\n".join(lines)


def make_case(batch, dim, seqlen, nstate, dtype, seed=0, with_z=True, h_init=False,
              delta_shift=0.0):
    return R.make_inputs(batch, dim, seqlen, nstate, seed=seed, dtype=dtype, with_z=with_z,
                         delta_shift=delta_shift, h_init=h_init)


def to_dev(case: dict, dev) -> dict:
    return {k: (None if v is None else v.to(dev).contiguous()) for k, v in case.items()}


class Lazy:
    """Evaluates fn() once, on first use (the oracle's magnitude runs)."""

    def __init__(self, fn):
        self._fn, self._v, self._done = fn, None, False

    def __call__(self):
        if not self._done:
            self._v, self._done = self._fn(), True
        return self._v

    def get(self, key):
        return lambda: self()[key]


def make_lm(seed=0, vocab=37, model_dim=16, state_dim=4, layers=2, bias=True, conv_bias=True,
            tie=True):
    """A small CausalLM (float32, CPU, eval mode, no dropout) with every
    parameter randomised -- norm weights and biases too, so no term of the
    model is trivially zero."""
    from ssm_mamba_amd.causal_lm import CausalLM, CausalLMConfig
    torch.manual_seed(seed)
    cfg = CausalLMConfig(vocab_size=vocab, model_dim=model_dim, state_dim=state_dim,
                         num_layers=layers, bias=bias, conv_bias=conv_bias, tie_embeddings=tie,
                         dropout_rate=0.0)
    with torch.device("cpu"):
        m = CausalLM(cfg).float()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("norm.weight") or (name.endswith(".bias") and "delta_proj" not in name):
                p.copy_(0.3 * torch.randn(p.shape, generator=g))
    return m.eval(), cfg


def lm_state64(model):
    """The model's state_dict as float64 CPU tensors, tied weights kept tied."""
    sd = {k: v.detach().to("cpu", torch.float64) for k, v in model.state_dict().items()}
    if model.lm_head.weight is model.embedding.weight:
        sd["lm_head.weight"] = sd["embedding.weight"]
    return sd
