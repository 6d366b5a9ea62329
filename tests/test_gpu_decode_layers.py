"""The layer chain (ssm_decode_layers: the decode step of every layer in one
persistent launch, workgroups handing activations to each other through
flagged buffer units instead of grid barriers) against the
per-layer fused kernels (logits, SSM states and conv windows over several
token steps; the chain sums the out-projection in K-slices and splits the
state update over thread pairs, so the two agree to rounding), for fp32 and
bf16, batch 1 to 4, with and without the optional biases, at small widths and
at the config-4 widths; repeat runs bit for bit; HIP-graph replays of the
chain against its eager steps bit for bit; and the chain's step against the
oracle's step chain."""
import pytest
import torch

from oracle import lm_ref as LR
from tests.helpers import assert_close, lm_state64, make_lm

pytestmark = pytest.mark.gpu


def _ids(batch, seqlen, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(3, vocab, (batch, seqlen), generator=g)
    for b in range(1, batch):
        ids[b, : 3 * b] = 0  # left padding of different lengths
    return ids


def _decode(m, ids, toks, chain, cuda):
    """Prefill, then one model step per token row; returns the logits and the
    final caches.  chain selects the layer chain or the per-layer kernels."""
    from ssm_mamba_amd import decode as DEC
    DEC.LAYER_CHAIN = chain
    try:
        with torch.no_grad():
            lengths = (ids != 0).sum(dim=1).to(cuda)
            m(ids.to(cuda), lengths, use_cache=True)
            logits = [m.step(t.to(cuda)).clone() for t in toks]
            states = torch.stack([l.ssm._ssm_hiddens.clone() for l in m.layers])
            windows = torch.stack([l.ssm._conv_context.clone() for l in m.layers])
    finally:
        DEC.LAYER_CHAIN = True
    return logits, states, windows


def _check_equal(a, b):
    for i, (x, y) in enumerate(zip(a[0], b[0])):
        assert torch.equal(x, y), f"logits of step {i} differ (max {float((x - y).abs().max()):.3g})"
    assert torch.equal(a[1], b[1]), "SSM states differ"
    assert torch.equal(a[2], b[2]), "conv windows differ"


def _close(got, ref, name, rtol, atol):
    g, r = got.double().cpu(), ref.double().cpu()
    err = (g - r).abs()
    bound = atol + rtol * r.abs()
    assert bool((err <= bound).all()), (
        f"{name}: max abs err {float(err.max()):.3g}, worst excess {float((err - bound).max()):.3g}")


def _check_close(a, b, dtype):
    """The chain against the per-layer kernels.  fp32: rounding-order
    differences only.  bf16: the activations between the kernels are bf16, so
    a one-ulp difference in one of them carries through the later layers and
    steps; the bound is the one the fused step meets against the op-by-op
    step (tests/test_gpu_lm.py)."""
    for i, (x, y) in enumerate(zip(a[0], b[0])):
        scale = float(y.abs().max())
        if dtype == torch.float32:
            _close(x, y, f"logits step {i}", rtol=1e-4, atol=1e-5 * scale)
        else:
            _close(x, y, f"logits step {i}", rtol=3e-2, atol=3e-2 * scale)
    tol = dict(rtol=1e-4, atol=1e-5) if dtype == torch.float32 else dict(rtol=3e-2, atol=3e-2)
    _close(a[1], b[1], "SSM states", **tol)
    _close(a[2].float(), b[2].float(), "conv windows", **tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch,model_dim,layers,kw", [
    (1, 128, 3, dict(bias=True, conv_bias=True)),
    (3, 128, 2, dict(bias=False, conv_bias=False)),
    (4, 256, 3, dict(bias=True, conv_bias=False)),
    (2, 128, 2, dict(bias=False, conv_bias=True)),
])
def test_chain_equals_per_layer_kernels(cuda, dtype, batch, model_dim, layers, kw):
    from ssm_mamba_amd import decode as DEC
    m, cfg = make_lm(seed=40 + batch, vocab=97, model_dim=model_dim, state_dim=16, layers=layers,
                     **kw)
    m = m.to(cuda, dtype)
    x = torch.zeros(batch, model_dim, device=cuda, dtype=dtype)
    m.allocate_cache(batch)
    with torch.no_grad():
        assert DEC.layers_supported(m.layers, x)
    ids = _ids(batch, 13, cfg.vocab_size, seed=41)
    toks = torch.randint(0, cfg.vocab_size, (6, batch), generator=torch.Generator().manual_seed(42))
    ref = _decode(m, ids, toks, chain=False, cuda=cuda)
    assert not m.__dict__.get("_layer_chains")
    got = _decode(m, ids, toks, chain=True, cuda=cuda)
    assert len(m.__dict__["_layer_chains"]) == 1, "the layer chain did not run"
    _check_close(got, ref, dtype)
    _check_equal(_decode(m, ids, toks, chain=True, cuda=cuda), got)


def test_chain_config4_widths(cuda):
    """Config-4 layer widths (d_model 1024, d_inner 2048, N 16, dt_rank 64,
    bf16, batch 4: 256 workgroups, one per CU), six layers."""
    m, cfg = make_lm(seed=50, vocab=211, model_dim=1024, state_dim=16, layers=6, bias=False,
                     conv_bias=True)
    m = m.to(cuda, torch.bfloat16)
    assert m.layers[0].ssm.delta_rank == 64
    ids = _ids(4, 9, cfg.vocab_size, seed=51)
    toks = torch.randint(0, cfg.vocab_size, (4, 4), generator=torch.Generator().manual_seed(52))
    ref = _decode(m, ids, toks, chain=False, cuda=cuda)
    got = _decode(m, ids, toks, chain=True, cuda=cuda)
    _check_close(got, ref, torch.bfloat16)
    _check_equal(_decode(m, ids, toks, chain=True, cuda=cuda), got)


def test_chain_graph_replays_match_eager(cuda):
    """The chain captured in a HIP graph: every replay equals the eager step
    from the same caches (the done counter returns to zero and the
    generation flag advances after each launch, so replays start clean),
    and the status check stays clear."""
    from ssm_mamba_amd import decode as DEC
    m, cfg = make_lm(seed=60, vocab=89, model_dim=256, state_dim=16, layers=4)
    m = m.to(cuda, torch.bfloat16)
    batch = 2
    ids = _ids(batch, 7, cfg.vocab_size, seed=61)
    with torch.no_grad():
        m(ids.to(cuda), (ids != 0).sum(dim=1).to(cuda), use_cache=True)
        caches0 = [(l.ssm._conv_context.clone(), l.ssm._ssm_hiddens.clone()) for l in m.layers]
        tok = torch.tensor([5, 17], device=cuda)
        x = m.embedding(tok)
        static_x = x.clone()
        # eager steps from the same caches
        eager = []
        for _ in range(3):
            static_x = DEC.layers_step(m, m.layers, static_x)
            eager.append(static_x.clone())
        DEC.layers_check(m)
        for l, (c, h) in zip(m.layers, caches0):
            l.ssm._conv_context.copy_(c)
            l.ssm._ssm_hiddens.copy_(h)
        inp = x.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            DEC.layers_step(m, m.layers, inp)  # warm-up (table and workspace exist)
        torch.cuda.current_stream().wait_stream(side)
        for l, (c, h) in zip(m.layers, caches0):
            l.ssm._conv_context.copy_(c)
            l.ssm._ssm_hiddens.copy_(h)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = DEC.layers_step(m, m.layers, inp)
        for i in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager[i]), f"replay {i} differs from the eager step"
            inp.copy_(out)
        DEC.layers_check(m)


def test_chain_failure_path(cuda):
    """The error word set from the host before a launch, as a timed-out wait
    leaves it (a flag the host sets: no wait is made to time out): every
    workgroup returns at its first check, so the launch changes no cache;
    layers_check raises and zero-fills the workspace; the next step then
    equals a fresh chain's step from the same caches, bit for bit."""
    from ssm_mamba_amd import decode as DEC
    m, cfg = make_lm(seed=62, vocab=89, model_dim=256, state_dim=16, layers=3)
    m = m.to(cuda, torch.bfloat16)
    ids = _ids(2, 7, cfg.vocab_size, seed=63)
    snap = lambda: [(l.ssm._conv_context.clone(), l.ssm._ssm_hiddens.clone()) for l in m.layers]
    with torch.no_grad():
        m(ids.to(cuda), (ids != 0).sum(dim=1).to(cuda), use_cache=True)
        x = m.embedding(torch.tensor([5, 17], device=cuda))
        DEC.layers_step(m, m.layers, x)  # a normal launch first (generation 1)
        DEC.layers_check(m)
        (chain,) = m.__dict__["_layer_chains"].values()
        caches0 = snap()
        err = chain.workspace[512:516]  # the error word (include/ssm_mamba.h)
        err.copy_(torch.tensor([1, 0, 0, 0], dtype=torch.uint8))
        DEC.layers_step(m, m.layers, x)
        torch.cuda.synchronize()
        for (c0, h0), (c1, h1) in zip(caches0, snap()):
            assert torch.equal(c0, c1) and torch.equal(h0, h1), "a launch ran past the error word"
        with pytest.raises(RuntimeError, match="timed out"):
            DEC.layers_check(m)
        assert int(chain.workspace.count_nonzero()) == 0, "the workspace was not cleared"
        got = DEC.layers_step(m, m.layers, x)
        DEC.layers_check(m)
        got_caches = snap()
        for l, (c, h) in zip(m.layers, caches0):
            l.ssm._conv_context.copy_(c)
            l.ssm._ssm_hiddens.copy_(h)
        fresh = DEC.LayerChain(m.layers, x)
        ref = fresh.step(m.layers, x)
        fresh.check()
    assert torch.equal(got, ref), "the step after the reset differs from a fresh chain's"
    for (c0, h0), (c1, h1) in zip(got_caches, snap()):
        assert torch.equal(c0, c1) and torch.equal(h0, h1)


def test_chain_step_matches_oracle(cuda):
    """fp32 model through the harness (the chain path) against the oracle's
    step chain in float64."""
    from ssm_mamba_amd import decode as DEC
    m, cfg = make_lm(seed=70, vocab=61, model_dim=64, state_dim=16, layers=3)
    m = m.to(cuda)
    assert m.layers[0].ssm.delta_rank == 4
    sd = lm_state64(m)
    ids = _ids(3, 15, cfg.vocab_size, seed=71)
    lengths = (ids != 0).sum(dim=1)
    toks = torch.randint(0, cfg.vocab_size, (5, 3), generator=torch.Generator().manual_seed(72))
    with torch.no_grad():
        m(ids.to(cuda), lengths.to(cuda), use_cache=True)
        got = [m.step(t.to(cuda)) for t in toks]
    assert m.__dict__.get("_layer_chains"), "the layer chain did not run"
    _, caches = LR.lm_forward(sd, ids, lengths, use_cache=True)
    W = sd["lm_head.weight"].detach().double().abs()
    for i, t in enumerate(toks):
        ex = {}
        ref, caches = LR.lm_step(sd, t, caches, extras=ex)
        # the fp32 bar, and where the head's terms cancel the float32
        # rounding term over their sizes (tests/helpers.py: C_CHAIN)
        assert_close(got[i], ref, torch.float32, f"chain step logits {i}",
                     ex["hidden"].abs() @ W.t())
    assert DEC.LAYER_CHAIN


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch,vocab", [(1, 8), (4, 50280), (3, 1000), (8, 4096)])
def test_pick_matches_torch_argmax(cuda, dtype, batch, vocab):
    """The greedy pick against torch.argmax on softmax outputs, with ties
    (equal maxima at several positions: the first wins) and NaNs (the first
    NaN wins, as in torch), plus its bookkeeping: tokens[:, min(pos, cols-1)]
    and pos + 1, the column clamped at the end."""
    from ssm_mamba_amd import decode as DEC
    g = torch.Generator().manual_seed(batch * vocab)
    logits = torch.randn(batch, vocab, generator=g)
    probs = torch.softmax(logits, dim=-1).to(dtype)
    if batch > 1:
        # row 1: the maximum also at later positions (a tie the first must win)
        j = int(probs[1].float().argmax())
        for k in (j + 3, vocab - 1):
            if k < vocab:
                probs[1, k] = probs[1, j]
    if batch > 2:
        probs[2, vocab // 3] = float("nan")
        probs[2, vocab // 2] = float("nan")
    probs = probs.to(cuda)
    ref = probs.argmax(dim=-1)
    cols = 5
    token = torch.zeros(batch, dtype=torch.int64, device=cuda)
    tokens = torch.full((batch, cols), -1, dtype=torch.int64, device=cuda)
    pos = torch.tensor([3], dtype=torch.int64, device=cuda)
    assert DEC.pick_supported(probs)
    for step in range(3):
        DEC.pick(probs, token, tokens, pos)
    torch.cuda.synchronize()
    assert torch.equal(token, ref), f"{token.tolist()} vs {ref.tolist()}"
    assert int(pos) == 6
    assert torch.equal(tokens[:, 3], ref) and torch.equal(tokens[:, 4], ref)
    assert bool((tokens[:, :3] == -1).all())
