"""Pins the causal-LM glue oracle (oracle/lm_ref.py) and checks the host side of
the model harness (ssm_mamba_amd.causal_lm) on the CPU.

The oracle's pieces are pinned by: torch's conv1d for the causal depthwise
conv; closed forms for RMSNorm; the prefill/step invariant (prefill of L
tokens then one step == prefill of L+1 tokens, which pins the conv window,
the state carry and the step path against the prefill path); a zero-B closed
form for the mixer; the zero-out-projection identity of a block; and the
reference's EOS rule on a model whose logits are forced flat.  No kernel is
called: the harness modules are only constructed here.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import lm_ref as LR
from tests.helpers import lm_state64, make_lm


@pytest.fixture(autouse=True)
def _float64_default():
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def tiny_sd(seed=0, **kw):
    m, cfg = make_lm(seed=seed, **kw)
    return lm_state64(m), cfg


def test_causal_conv_matches_torch_conv1d():
    g = torch.Generator().manual_seed(0)
    for k in (1, 2, 4, 5):
        x = torch.randn(2, 6, 11, generator=g)
        w = torch.randn(6, 1, k, generator=g)
        b = torch.randn(6, generator=g)
        ref = F.conv1d(x, w, b, padding=k - 1, groups=6)[..., :11]
        torch.testing.assert_close(LR.causal_conv(x, w, b), ref, rtol=1e-12, atol=1e-12)
    # sequence shorter than the kernel
    x = torch.randn(1, 3, 2, generator=g)
    w = torch.randn(3, 1, 4, generator=g)
    torch.testing.assert_close(LR.causal_conv(x, w, None),
                               F.conv1d(x, w, None, padding=3, groups=3)[..., :2])


def test_rms_norm_closed_forms():
    w = torch.tensor([0.5, -0.25, 0.0, 2.0])
    c = -3.0
    x = torch.full((1, 4), c)
    want = math.copysign(1.0, c) * abs(c) / math.sqrt(c * c + 1e-6) * (1.0 + w)
    torch.testing.assert_close(LR.rms_norm(x, w)[0], want)
    # scale invariance (eps aside) and the unit-RMS output for w = 0
    g = torch.Generator().manual_seed(3)
    y = torch.randn(5, 64, generator=g)
    torch.testing.assert_close(LR.rms_norm(7.0 * y, w.new_zeros(64), eps=0.0),
                               LR.rms_norm(y, w.new_zeros(64), eps=0.0))
    r = LR.rms_norm(y, y.new_zeros(64), eps=0.0)
    torch.testing.assert_close(r.pow(2).mean(-1), torch.ones(5))


@pytest.mark.parametrize("bias", [False, True])
def test_prefill_then_step_equals_longer_prefill(bias):
    sd, cfg = tiny_sd(seed=2, bias=bias, conv_bias=bias)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(3, cfg.vocab_size, (2, 13), generator=g)
    full, _ = LR.lm_forward(sd, ids)
    pre, caches = LR.lm_forward(sd, ids[:, :9], use_cache=True)
    torch.testing.assert_close(pre, full[:, :9])
    for t in range(9, 13):
        logits, caches = LR.lm_step(sd, ids[:, t], caches)
        torch.testing.assert_close(logits, full[:, t], rtol=1e-10, atol=1e-10)


def test_prefill_shorter_than_conv_window_then_steps():
    sd, cfg = tiny_sd(seed=4)
    ids = torch.tensor([[5, 9, 11, 4, 7, 8]])
    full, _ = LR.lm_forward(sd, ids)
    _, caches = LR.lm_forward(sd, ids[:, :2], use_cache=True)   # window reaches before t = 0
    for t in range(2, 6):
        logits, caches = LR.lm_step(sd, ids[:, t], caches)
        torch.testing.assert_close(logits, full[:, t], rtol=1e-10, atol=1e-10)


def test_mixer_with_zero_B_is_skip_path_only():
    """B = 0 leaves the state at zero, so the scan output is D*x*silu(gate)."""
    sd, cfg = tiny_sd(seed=6)
    p = LR.layer_params(sd, 0)
    N, R = cfg.state_dim, sd["layers.0.ssm.delta_proj.weight"].shape[1]
    p["ssm.ssm_param_proj.weight"][R:R + N] = 0.0
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 10, cfg.model_dim, generator=g)
    y, last, _ = LR.mamba_forward(p, x, N, R)
    inner = p["ssm.input_proj.weight"].shape[0] // 2
    xz = x @ p["ssm.input_proj.weight"].t() + p["ssm.input_proj.bias"]
    xs, gate = xz[..., :inner], xz[..., inner:]
    conv = F.conv1d(xs.transpose(1, 2), p["ssm.conv.weight"], p["ssm.conv.bias"], padding=3,
                    groups=inner)[..., :10].transpose(1, 2)
    xc = F.silu(conv)
    want = (p["ssm.D"] * xc * F.silu(gate)) @ p["ssm.out_proj.weight"].t() + p["ssm.out_proj.bias"]
    torch.testing.assert_close(y, want)
    assert float(last.abs().max()) == 0.0


def test_block_with_zero_out_projection_is_identity():
    sd, cfg = tiny_sd(seed=7, bias=False, layers=1, tie=False)
    sd["layers.0.ssm.out_proj.weight"].zero_()
    sd["norm.weight"].zero_()
    ids = torch.tensor([[3, 4, 5, 6]])
    logits, _ = LR.lm_forward(sd, ids)
    x = sd["embedding.weight"][ids]
    want = LR.rms_norm(x, sd["norm.weight"]) @ sd["lm_head.weight"].t()
    torch.testing.assert_close(logits, want)


def test_generate_stops_at_eos_and_masks_after_it():
    """Flat logits (final norm scale 1 + w = 0) make argmax pick token 0; with
    eos = 0 every row ends after one new token and everything from a row's
    first 0 on becomes 0, as in models/causal_lm.py:123-133."""
    sd, cfg = tiny_sd(seed=8)
    sd["norm.weight"].fill_(-1.0)
    ids = torch.tensor([[4, 0, 6, 7], [5, 6, 7, 8]])
    out = LR.generate(sd, ids, max_new_tokens=5, pad_id=1, eos_id=0)
    assert out.tolist() == [[4, 0, 0, 0, 0], [5, 6, 7, 8, 0]]
    # without an EOS hit the loop runs to max_new_tokens
    out = LR.generate(sd, ids, max_new_tokens=3, pad_id=1, eos_id=2)
    assert out.shape == (2, 7) and out[:, 4:].eq(0).all()


REFERENCE_PARAM_NAMES = {
    # modules/rms_norm.py:8, modules/mamba.py:35-79, modules/block.py:29-48,
    # models/causal_lm.py:38-63
    "embedding.weight", "norm.weight", "lm_head.weight",
    "layers.0.norm.weight",
    "layers.0.ssm.input_proj.weight", "layers.0.ssm.conv.weight",
    "layers.0.ssm.ssm_param_proj.weight", "layers.0.ssm.delta_proj.weight",
    "layers.0.ssm.delta_proj.bias", "layers.0.ssm.log_A", "layers.0.ssm.D",
    "layers.0.ssm.out_proj.weight",
}


def test_harness_parameter_names_shapes_and_init():
    from ssm_mamba_amd.causal_lm import CausalLM, CausalLMConfig
    torch.manual_seed(0)
    cfg = CausalLMConfig(vocab_size=100, model_dim=64, num_layers=1)
    m = CausalLM(cfg)
    sd = m.state_dict()
    assert set(sd) == REFERENCE_PARAM_NAMES
    ssm = m.layers[0].ssm
    assert ssm.inner_dim == 128 and ssm.delta_rank == 4
    assert tuple(sd["layers.0.ssm.input_proj.weight"].shape) == (256, 64)
    assert tuple(sd["layers.0.ssm.conv.weight"].shape) == (128, 1, 4)
    assert tuple(sd["layers.0.ssm.ssm_param_proj.weight"].shape) == (4 + 32, 128)
    assert tuple(sd["layers.0.ssm.delta_proj.weight"].shape) == (128, 4)
    assert m.lm_head.weight is m.embedding.weight
    torch.testing.assert_close(-torch.exp(ssm.log_A.float()),
                               -torch.arange(1, 17, dtype=torch.float32).expand(128, 16))
    assert float(ssm.D.detach().min()) == 1.0 == float(ssm.D.detach().max())
    assert float(m.norm.weight.detach().abs().max()) == 0.0
    # delta_proj bias is softplus^-1 of a step in [1e-3, 0.1]
    dt = F.softplus(ssm.delta_proj.bias.detach().double())
    assert float(dt.min()) >= 1e-3 * (1 - 1e-5) and float(dt.max()) <= 0.1 * (1 + 1e-5)
    bound = 4 ** -0.5
    assert float(ssm.delta_proj.weight.detach().abs().max()) <= bound
    with pytest.raises(RuntimeError):
        ssm.step(torch.zeros(1, 64))                  # no caches yet
