"""Shared helpers for the parity tests (HIP path vs the CPU oracle)."""
from __future__ import annotations

import torch

from oracle import scan_ref as R

# Tolerances stated by the task for this path: fp32 rtol 1e-4 / atol 1e-5;
# bf16 inputs with fp32 accumulation rtol 2e-2 / atol 5e-3 (outputs and grads).
TOL = {
    torch.float32: dict(rtol=1e-4, atol=1e-5),
    torch.bfloat16: dict(rtol=2e-2, atol=5e-3),
}


def assert_close(got: torch.Tensor, ref: torch.Tensor, dtype, name: str, scale_atol: bool = False):
    """Compare a GPU result with the float64 oracle.  With scale_atol the
    absolute tolerance is taken relative to the tensor's RMS (used for
    quantities that are long fp32 sums of O(1) terms)."""
    tol = dict(TOL[dtype])
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    if scale_atol:
        tol["atol"] = tol["atol"] * max(1.0, float(r.pow(2).mean().sqrt()))
    err = (g - r).abs()
    bound = tol["atol"] + tol["rtol"] * r.abs()
    bad = err > bound
    if bad.any():
        i = int(torch.argmax((err - bound).flatten()))
        raise AssertionError(
            f"{name}: {int(bad.sum())}/{err.numel()} elements out of tolerance {tol}; "
            f"worst at flat index {i}: got {g.flatten()[i].item():.8g} ref {r.flatten()[i].item():.8g}; "
            f"max abs err {err.max().item():.3g}")


def make_case(batch, dim, seqlen, nstate, dtype, seed=0, with_z=True, h_init=False,
              delta_shift=0.0):
    return R.make_inputs(batch, dim, seqlen, nstate, seed=seed, dtype=dtype, with_z=with_z,
                         delta_shift=delta_shift, h_init=h_init)


def to_dev(case: dict, dev) -> dict:
    return {k: (None if v is None else v.to(dev).contiguous()) for k, v in case.items()}
