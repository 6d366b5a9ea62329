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
