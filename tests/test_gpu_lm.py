"""GPU parity of the causal-LM harness (ssm_mamba_amd.causal_lm) against the CPU
oracle of the reference's model code (oracle/lm_ref.py): prefill logits with
and without padding, the decode step chain, greedy generation (HIP-graph and
eager paths), graph replays against eager steps, bf16 weights, and parameter
gradients of a training step through the HIP scan backward."""
import pytest
import torch

from oracle import lm_ref as LR
from tests.helpers import assert_close, lm_state64, make_lm

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


@pytest.mark.parametrize("pads", [False, True])
def test_forward_last_is_the_row_at_lengths_minus_1(cuda, pads):
    """forward_last (the prefill of generate: norm and LM head on one row per
    sequence) against the oracle's full logits at lengths - 1, the rows the
    reference's generate keeps (an empty row's index -1 wraps to the end)."""
    m, cfg = make_lm(seed=1, vocab=53, model_dim=32, state_dim=16, layers=2)
    sd = lm_state64(m)
    m = m.to(cuda)
    ids = _ids(3, 37, cfg.vocab_size, seed=2, pads=pads)
    lengths = (ids != cfg.pad_token_id).sum(dim=1)
    with torch.no_grad():
        got = m.forward_last(ids.to(cuda), lengths.to(cuda))
    ref, _ = LR.lm_forward(sd, ids, lengths)
    assert got.shape == (3, cfg.vocab_size)
    _close(got, ref[torch.arange(3), lengths - 1], "last-position logits", **F32)


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
        pick = lambda lg: torch.softmax(lg, dim=-1).argmax(-1)
        tok = pick(m.forward_last(ids, lengths, use_cache=True))
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


@pytest.mark.parametrize("pads", [False, True])
def test_training_gradients_fp32(cuda, pads):
    """Parameter gradients of sum(logits * r) through the HIP scan backward,
    against float64 autograd through the oracle model, at the stated fp32
    bar.  With left-padded prompts (``lengths``) the oracle follows the
    reference's training rule: the scan drops the upstream gradient of its
    padded outputs, the gate and the other paths do not."""
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
        assert_close(names[k].grad, sd[k].grad, torch.float32, f"grad {k}")


@pytest.mark.parametrize("fold", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch,kw", [
    (1, dict(bias=True, conv_bias=True)),
    (3, dict(bias=False, conv_bias=False)),
    (8, dict(bias=True, conv_bias=False)),
])
def test_fused_decode_matches_eager_and_oracle(cuda, dtype, batch, kw, fold):
    """The fused decode kernels per layer (three with the x-projection folded
    into its neighbours, four without) and the fused LM head against the
    op-by-op step and the oracle's step chain."""
    from ssm_mamba_amd import decode as DEC
    m, cfg = make_lm(seed=20 + batch, vocab=67, model_dim=64, state_dim=16, layers=2, **kw)
    m = m.to(cuda, dtype)
    ssm0 = m.layers[0].ssm
    assert DEC.xproj_blocks(ssm0.inner_dim, ssm0.ssm_param_proj.weight.shape[0]) == 8
    sd = lm_state64(m)
    ids = _ids(batch, 19, cfg.vocab_size, seed=21)
    lengths = (ids != cfg.pad_token_id).sum(dim=1)
    toks = torch.randint(0, cfg.vocab_size, (5, batch), generator=torch.Generator().manual_seed(22))
    outs = {}
    for fused in (True, False):
        DEC.ENABLED = fused
        DEC.FOLD_XPROJ = fold
        try:
            with torch.no_grad():
                m(ids.to(cuda), lengths.to(cuda), use_cache=True)
                outs[fused] = [m.step(t.to(cuda)).float() for t in toks]
                outs[(fused, "state")] = torch.stack([l.ssm._ssm_hiddens.clone() for l in m.layers])
                outs[(fused, "ctx")] = torch.stack([l.ssm._conv_context.float() for l in m.layers])
        finally:
            DEC.ENABLED = True
            DEC.FOLD_XPROJ = True
    _, caches = LR.lm_forward(sd, ids, lengths, use_cache=True)
    if dtype == torch.float32:
        tol = dict(rtol=1e-3, atol=1e-4)
    else:
        tol = dict(rtol=3e-2, atol=3e-2 * float(outs[False][0].abs().max()))
    for i, t in enumerate(toks):
        ref, caches = LR.lm_step(sd, t, caches)
        _close(outs[True][i], ref, f"fused step {i}", **tol)
        _close(outs[True][i], outs[False][i], f"fused vs eager step {i}", **tol)
    _close(outs[(True, "state")], torch.stack([c[1] for c in caches]), "fused state", **tol)
    _close(outs[(True, "ctx")], torch.stack([c[0] for c in caches]), "fused window",
           rtol=tol["rtol"], atol=1e-6 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch,dim,rank,nstate", [
    (1, 16, 3, 4),        # one block, params_dim 11 (padded to 12)
    (3, 128, 4, 16),
    (4, 2048, 64, 16),    # the 370M-class layer
    (8, 1024, 160, 16),   # params_dim 192 (2.8B-class rank)
    (2, 48, 248, 4),      # params_dim 256, the limit; rank past the register path
])
def test_folded_xproj(cuda, dtype, batch, dim, rank, nstate):
    """The x-projection folded into the in-projection (fp32 partials per
    16-channel block) and the state update (fixed-order sum): the partials
    against float64 products of the kernel's own xc, zero padding, the
    update's output and state against the unfolded chain (in-projection,
    GEMV, update), and bit-identical repeats."""
    from ssm_mamba_amd import decode as DEC
    g = torch.Generator().manual_seed(dim + rank + batch)
    K, width = 64, 4
    nout = rank + 2 * nstate
    r = lambda *s, scale=1.0: (scale * torch.randn(*s, generator=g)).to(dtype).to(cuda)
    W_in, x, nw = r(2 * dim, K, scale=0.2), r(batch, K), r(K, scale=0.3)
    b_in, cw, cb = r(2 * dim, scale=0.1), r(dim, width, scale=0.5), r(dim, scale=0.1)
    window = r(batch, dim, width - 1)
    W_x, W_dt, dtb = r(nout, dim, scale=0.1), r(dim, rank, scale=0.2), r(dim, scale=0.5)
    log_A = (torch.rand(dim, nstate, generator=g) * 2).to(dtype).to(cuda)
    D = r(dim)
    state = torch.randn(batch, dim, nstate, generator=g).to(cuda)
    nparts = DEC.xproj_blocks(dim, nout)
    assert nparts == dim // 16
    with torch.no_grad():
        w1, s1 = window.clone(), state.clone()
        xz1, xc1 = DEC.in_proj_conv(W_in, x, nw, 1e-6, b_in, cw, cb, w1)
        params = DEC.gemv(W_x, xc1)
        y1 = DEC.ssm_step(params, rank, W_dt, dtb, log_A, D, xc1, xz1, s1)
        runs = []
        for _ in range(2):
            w2, s2 = window.clone(), state.clone()
            xz2, xc2, part = DEC.in_proj_conv(W_in, x, nw, 1e-6, b_in, cw, cb, w2, x_proj_weight=W_x)
            y2 = DEC.ssm_step(part, rank, W_dt, dtb, log_A, D, xc2, xz2, s2)
            runs.append((xz2, xc2, part, y2, s2, w2))
    xz2, xc2, part, y2, s2, w2 = runs[0]
    for a, b in zip(runs[0], runs[1]):
        assert torch.equal(a, b), "folded decode step is not bit-reproducible"
    assert part.shape == (nparts, batch, (nout + 3) // 4 * 4) and part.dtype == torch.float32
    assert torch.equal(part[..., nout:], torch.zeros_like(part[..., nout:]))
    ref = torch.einsum("jpc,bpc->pbj", W_x.double().cpu().view(nout, nparts, 16),
                       xc2.double().cpu().view(batch, nparts, 16))
    _close(part[..., :nout], ref, "partials", rtol=1e-5, atol=1e-6)
    same = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=1e-2, atol=1e-2)
    _close(xz2, xz1, "xz", **same)
    _close(xc2, xc1, "xc", **same)
    _close(w2, w1, "window", **same)
    # the update sees round_T(sum of partials) for the GEMV's round_T(W_x @ xc):
    # equal up to the last bit of those roundings
    step = dict(rtol=1e-4, atol=1e-4) if dtype == torch.float32 else dict(rtol=3e-2, atol=3e-2)
    _close(s2, s1, "state", **step)
    _close(y2, y1, "y", rtol=step["rtol"], atol=step["atol"] * max(1.0, float(y1.abs().max())))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch", [1, 2, 5, 8])
@pytest.mark.parametrize("out_dim,in_dim", [(1, 8), (37, 64), (300, 1032), (64, 4096)])
def test_decode_gemv(cuda, dtype, batch, out_dim, in_dim):
    from ssm_mamba_amd import decode as DEC
    g = torch.Generator().manual_seed(out_dim + in_dim + batch)
    W = torch.randn(out_dim, in_dim, generator=g).to(dtype)
    x = torch.randn(batch, in_dim, generator=g).to(dtype)
    nw = (0.3 * torch.randn(in_dim, generator=g)).to(dtype)
    bias = torch.randn(out_dim, generator=g).to(dtype)
    res = torch.randn(batch, out_dim, generator=g).to(dtype)
    d = lambda t: t.to(cuda)
    with torch.no_grad():
        for use_norm in (False, True):
            for use_extra in (False, True):
                got = DEC.gemv(d(W), d(x), norm_weight=d(nw) if use_norm else None, eps=1e-6,
                               bias=d(bias) if use_extra else None,
                               residual=d(res) if use_extra else None)
                v = x.double()
                if use_norm:
                    v = LR.rms_norm(v, nw.double())
                ref = v @ W.double().t()
                if use_extra:
                    ref = ref + bias.double() + res.double()
                scale = float(ref.abs().max())
                if dtype == torch.float32:
                    _close(got, ref, "gemv", rtol=1e-4, atol=1e-5 * max(1.0, scale))
                else:
                    _close(got, ref, "gemv", rtol=1e-2, atol=1e-2 * max(1.0, scale))


def test_fused_decode_falls_back_outside_its_limits(cuda):
    """Batch 9 exceeds the fused kernels' limit: the step takes the op-by-op
    path and still matches the oracle."""
    from ssm_mamba_amd import decode as DEC
    m, cfg = make_lm(seed=30, vocab=29, model_dim=32, state_dim=16, layers=1)
    m = m.to(cuda)
    sd = lm_state64(m)
    ids = _ids(9, 11, cfg.vocab_size, seed=31, pads=False)
    with torch.no_grad():
        m(ids.to(cuda), use_cache=True)
        assert not DEC.block_step_supported(m.layers[0].ssm, torch.zeros(9, 32, device=cuda),
                                            m.layers[0].norm.weight)
        got = m.step(ids[:, 0].to(cuda))
    _, caches = LR.lm_forward(sd, ids, use_cache=True)
    ref, _ = LR.lm_step(sd, ids[:, 0], caches)
    _close(got, ref, "batch-9 step", **F32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch,ch,seqlen", [(1, 8, 1), (2, 64, 37), (3, 1024, 256), (2, 100, 130),
                                              (1, 2048, 77), (4, 1024, 2048)])
def test_rms_norm_channel_major(cuda, dtype, batch, ch, seqlen):
    """The channel-major RMSNorm kernel against the oracle's RMSNorm over the
    channel axis, including odd lengths (element path) and an offset view."""
    from ssm_mamba_amd.causal_lm import rms_norm_cm
    g = torch.Generator().manual_seed(batch * ch + seqlen)
    x = (torch.randn(batch, ch, seqlen + 1, generator=g) * 3).to(dtype)
    w = (0.3 * torch.randn(ch, generator=g)).to(dtype)
    for xs in (x[..., :seqlen], x[..., 1:]):
        xs = xs.contiguous()
        got = rms_norm_cm(xs.to(cuda), w.to(cuda), 1e-6)
        ref = LR.rms_norm(xs.double().transpose(1, 2), w.double()).transpose(1, 2)
        tol = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=1e-2, atol=1e-2)
        _close(got, ref, "rms_norm_cm", **tol)
    # an odd element offset exercises the unpaired path
    flat = torch.randn(batch * ch * seqlen + 1, generator=g).to(dtype).to(cuda)
    xo = flat[1:].view(batch, ch, seqlen)
    got = rms_norm_cm(xo, w.to(cuda), 1e-6)
    ref = LR.rms_norm(xo.cpu().double().transpose(1, 2), w.double()).transpose(1, 2)
    tol = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=1e-2, atol=1e-2)
    _close(got, ref, "rms_norm_cm offset", **tol)
