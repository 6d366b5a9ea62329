"""GPU parity of the causal-LM harness (ssm_mamba_amd.causal_lm) against the CPU
oracle of the reference's model code (oracle/lm_ref.py): prefill logits with
and without padding, the decode step chain, greedy generation (HIP-graph and
eager paths), graph replays against eager steps, bf16 weights, and parameter
gradients of a training step through the HIP scan backward."""
import pytest
import torch

from oracle import lm_ref as LR
from tests.helpers import lm_state64, make_lm

pytestmark = pytest.mark.gpu

# fp32 model: long chains of fp32 GEMMs and scans against float64
F32 = dict(rtol=1e-3, atol=1e-4)


def _ids(batch, seqlen, vocab, seed, pads=True):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(3, vocab, (batch, seqlen), generator=g)
    if pads:
        # left-padded prompts of different lengths, one of them empty
        for b in range(1, batch):
            ids[b, : min(seqlen, 5 * b + (seqlen if b == batch - 1 else 0))] = 0
    return ids


def _close(got, ref, name, rtol, atol):
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    err = (g - r).abs()
    bound = atol + rtol * r.abs()
    assert bool((err <= bound).all()), (
        f"{name}: max abs err {err.max().item():.3g}, worst excess "
        f"{(err - bound).max().item():.3g} (rtol {rtol}, atol {atol})")


@pytest.mark.parametrize("pads", [False, True])
def test_prefill_logits_fp32(cuda, pads):
    m, cfg = make_lm(seed=1, vocab=53, model_dim=32, state_dim=16, layers=2)
    sd = lm_state64(m)
    m = m.to(cuda)
    ids = _ids(3, 37, cfg.vocab_size, seed=2, pads=pads)
    lengths = (ids != cfg.pad_token_id).sum(dim=1)
    with torch.no_grad():
        got = m(ids.to(cuda), lengths.to(cuda) if pads else None)
    ref, _ = LR.lm_forward(sd, ids, lengths if pads else None)
    _close(got, ref, "logits", **F32)


def test_prefill_then_steps_fp32(cuda):
    m, cfg = make_lm(seed=3, vocab=41, model_dim=32, state_dim=16, layers=3, bias=False,
                     conv_bias=False)
    sd = lm_state64(m)
    m = m.to(cuda)
    ids = _ids(2, 21, cfg.vocab_size, seed=4)
    lengths = (ids != cfg.pad_token_id).sum(dim=1)
    with torch.no_grad():
        got = m(ids.to(cuda), lengths.to(cuda), use_cache=True)
    ref, caches = LR.lm_forward(sd, ids, lengths, use_cache=True)
    _close(got, ref, "prefill logits", **F32)
    for layer, (ctx, state) in zip(m.layers, caches):
        _close(layer.ssm._conv_context, ctx, "conv window", **F32)
        _close(layer.ssm._ssm_hiddens, state, "ssm state", **F32)
    g = torch.Generator().manual_seed(9)
    for t in range(6):
        tok = torch.randint(0, cfg.vocab_size, (2,), generator=g)
        with torch.no_grad():
            got = m.step(tok.to(cuda))
        ref, caches = LR.lm_step(sd, tok, caches)
        _close(got, ref, f"step {t} logits", **F32)


def test_generate_matches_reference_loop(cuda):
    m, cfg = make_lm(seed=5, vocab=29, model_dim=32, state_dim=16, layers=2)
    sd = lm_state64(m)
    m = m.to(cuda)
    ids = _ids(3, 17, cfg.vocab_size, seed=6)
    ref = LR.generate(sd, ids, max_new_tokens=20, pad_id=cfg.pad_token_id,
                      eos_id=cfg.eos_token_id)
    graph = m.generate(ids.to(cuda), max_new_tokens=20)
    eager = m.generate(ids.to(cuda), max_new_tokens=20, use_graph=False)
    assert eager.cpu().tolist() == ref.tolist()
    assert graph.cpu().tolist() == ref.tolist()
    # a second prompt through the same captured graph
    ids2 = _ids(3, 17, cfg.vocab_size, seed=7)
    ref2 = LR.generate(sd, ids2, max_new_tokens=20, pad_id=cfg.pad_token_id,
                       eos_id=cfg.eos_token_id)
    assert m.generate(ids2.to(cuda), max_new_tokens=20).cpu().tolist() == ref2.tolist()


def test_generate_stops_when_every_row_hit_eos(cuda):
    m, cfg = make_lm(seed=8, vocab=31, model_dim=32, state_dim=16, layers=1)
    with torch.no_grad():
        m.norm.weight.fill_(-1.0)        # flat logits: argmax is token 0
    m.config.eos_token_id = 0
    m.config.pad_token_id = 1
    m = m.to(cuda)
    ids = torch.tensor([[4, 0, 6, 7], [5, 6, 7, 8]])
    for use_graph in (True, False):
        out = m.generate(ids.to(cuda), max_new_tokens=5, use_graph=use_graph)
        assert out.cpu().tolist() == [[4, 0, 0, 0, 0], [5, 6, 7, 8, 0]]


def test_graph_replays_match_eager_steps(cuda):
    """Every replay of the captured step, with eager work and synchronisation in
    between, equals the eager step chain from the same prefill."""
    m, cfg = make_lm(seed=10, vocab=47, model_dim=64, state_dim=16, layers=2)
    m = m.to(cuda)
    ids = _ids(2, 33, cfg.vocab_size, seed=11).to(cuda)
    lengths = (ids != cfg.pad_token_id).sum(dim=1)
    steps = 7
    dec = m.decoder(2, steps + 1)
    dec.capture()
    with torch.no_grad():
        logits = m(ids, lengths, use_cache=True)
        pick = lambda lg: torch.softmax(lg, dim=-1).argmax(-1)
        tok = pick(logits[torch.arange(2, device=cuda), lengths - 1])
        eager_tokens = [tok]
        eager_states = []
        for _ in range(steps):
            tok = pick(m.step(tok))
            eager_tokens.append(tok)
            eager_states.append(torch.stack([l.ssm._ssm_hiddens.clone() for l in m.layers]))
    dec.prefill(ids, lengths)
    for i in range(steps):
        dec.replay(1)
        torch.cuda.synchronize()
        junk = torch.randn(4096, device=cuda).sum()     # unrelated eager work between replays
        state = torch.stack([l.ssm._ssm_hiddens for l in m.layers])
        assert torch.equal(dec.tokens[:, i + 1], eager_tokens[i + 1]), f"replay {i}"
        torch.testing.assert_close(state, eager_states[i], rtol=1e-6, atol=1e-6)
        assert torch.isfinite(junk)
    assert torch.equal(dec.tokens[:, 0], eager_tokens[0])


def test_bf16_weights_close_to_oracle(cuda):
    m, cfg = make_lm(seed=12, vocab=61, model_dim=64, state_dim=16, layers=2)
    m = m.to(cuda, torch.bfloat16)
    sd = lm_state64(m)          # the oracle sees the bf16-rounded weights
    ids = _ids(2, 40, cfg.vocab_size, seed=13)
    lengths = (ids != cfg.pad_token_id).sum(dim=1)
    with torch.no_grad():
        got = m(ids.to(cuda), lengths.to(cuda), use_cache=True)
        assert got.dtype == torch.bfloat16
    ref, caches = LR.lm_forward(sd, ids, lengths, use_cache=True)
    scale = float(ref.abs().max())
    _close(got, ref, "bf16 logits", rtol=3e-2, atol=3e-2 * scale)
    tok = torch.tensor([5, 9])
    with torch.no_grad():
        got = m.step(tok.to(cuda))
    ref, _ = LR.lm_step(sd, tok, caches)
    _close(got, ref, "bf16 step logits", rtol=3e-2, atol=3e-2 * scale)


def test_training_gradients_fp32(cuda):
    """Parameter gradients of sum(logits * r) through the HIP scan backward,
    against float64 autograd through the oracle model.  Unpadded: with
    ``lengths`` the scan's backward ignores the upstream gradient at padded
    positions (the reference's rule, covered by the operator tests), so the
    model gradient is then not the autograd gradient of the forward."""
    pads = False
    m, cfg = make_lm(seed=14, vocab=23, model_dim=32, state_dim=16, layers=2)
    sd = lm_state64(m)
    for v in sd.values():
        v.requires_grad_(True)
    m = m.to(cuda).train()
    ids = _ids(2, 29, cfg.vocab_size, seed=15, pads=pads)
    lengths = (ids != cfg.pad_token_id).sum(dim=1) if pads else None
    r = torch.randn(2, 29, cfg.vocab_size, generator=torch.Generator().manual_seed(16))
    got = m(ids.to(cuda), None if lengths is None else lengths.to(cuda))
    (got * r.to(cuda)).sum().backward()
    ref, _ = LR.lm_forward(sd, ids, lengths)
    (ref * r.double()).sum().backward()
    names = dict(m.named_parameters())
    for k in ["embedding.weight", "norm.weight", "layers.0.norm.weight",
              "layers.0.ssm.input_proj.weight", "layers.0.ssm.input_proj.bias",
              "layers.0.ssm.conv.weight", "layers.0.ssm.conv.bias",
              "layers.1.ssm.ssm_param_proj.weight", "layers.1.ssm.delta_proj.weight",
              "layers.1.ssm.delta_proj.bias", "layers.0.ssm.log_A", "layers.1.ssm.D",
              "layers.1.ssm.out_proj.weight"]:
        gr = sd[k].grad
        rms = float(gr.pow(2).mean().sqrt())
        _close(names[k].grad, gr, f"grad {k}", rtol=2e-3, atol=2e-4 * max(rms, 1e-3))
