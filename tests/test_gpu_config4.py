"""BASELINE config 4 (the 48-layer causal LM at d_model 1024, bf16) checked at
its widths:

* two layers at the config-4 widths (d_model 1024, d_inner 2048, N 16,
  dt_rank 64, vocab 50280, bf16, the reference's random init) against the
  float64 oracle of the reference's model code (oracle/lm_ref.py): a 4 x 2048
  prefill with pad-derived lengths (left padding), the logits at a subset of
  positions, every layer's conv window and state, then 8 decode steps;
* the full 48-layer model: 128 greedy steps replayed from the captured HIP
  graph equal 128 eager steps bit for bit (tokens, states, windows), and
  prefill(L) followed by one step matches prefill(L + 1).

Model-level tolerance: the stated bf16 bar (rtol 2e-2, atol 5e-3), plus, where
the terms of the last operation cancel, C_MODEL * 2^-8 * (sum of their |terms|)
with C_MODEL = 1: the last operation's input is stored in bf16, one rounding
of relative size 2^-8 per element, and its float32 sum over K <= 1024 terms
adds at most K * 2^-24 <= 2^-14 of the same sum of |terms|, a 64th of it,
which the rounding up of the constant covers.  Errors the layers before it
leave in that input are not budgeted separately: the check asserts that they
stay below one bf16 rounding of the input, which makes it a test of the
layers too.  Greedy tokens: wherever the oracle's top two logits differ by
more than the bounds of both, the HIP path's argmax must be the oracle's."""
import pytest
import torch

from oracle import lm_ref as LR
from tests.helpers import EPS_BF16, assert_close, lm_state64

pytestmark = pytest.mark.gpu

C4 = dict(vocab_size=50280, model_dim=1024, state_dim=16, dropout_rate=0.0)
BF16 = torch.bfloat16
# bf16 roundings of the last operation's input (see the module docstring)
C_MODEL = 1


def _model(layers, seed, dev):
    from ssm_mamba_amd.causal_lm import CausalLM, CausalLMConfig
    torch.manual_seed(seed)
    cfg = CausalLMConfig(**C4, num_layers=layers)
    with torch.device("cpu"):
        m = CausalLM(cfg)
    return m.to(dev, BF16).eval(), cfg


def _ids(batch, seqlen, vocab, seed, pads=(0, 300, 0, 1500)):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(1, vocab, (batch, seqlen), generator=g)
    for b, n in enumerate(pads[:batch]):
        ids[b, :n] = 0  # left padding with the pad id; lengths count the rest
    return ids


def _head_mag(hidden, W):
    """sum_k |hidden_k| |W_jk|: the sizes of the LM head's terms."""
    return hidden.abs().double() @ W.detach().double().abs().t().cpu()


def _check_greedy(got, ref, mag, name):
    """Where the oracle's best logit beats its second by more than the two
    elements' bounds together, the HIP path's argmax is the oracle's."""
    from oracle import scan_ref as R
    from tests.helpers import TOL
    g = got.detach().double().cpu().reshape(-1, got.shape[-1])
    r = ref.detach().double().cpu().reshape(-1, ref.shape[-1])
    t = TOL[BF16]
    bound = R.error_bound(r, mag.reshape(-1, mag.shape[-1]), t["rtol"], t["atol"], C_MODEL,
                          EPS_BF16)
    top2 = r.topk(2, dim=-1)
    i1, i2 = top2.indices[:, 0], top2.indices[:, 1]
    rows = torch.arange(r.shape[0])
    decided = (top2.values[:, 0] - top2.values[:, 1]) > bound[rows, i1] + bound[rows, i2]
    assert int(decided.sum()) > 0, f"{name}: no row has a decided argmax"
    same = g.argmax(dim=-1) == i1
    assert bool(same[decided].all()), (
        f"{name}: argmax differs at rows {torch.nonzero(decided & ~same).flatten().tolist()}")
    print(f"{name}: greedy argmax checked at {int(decided.sum())} of {r.shape[0]} rows", flush=True)


def test_config4_two_layers_vs_oracle(cuda):
    m, cfg = _model(2, seed=40, dev=cuda)
    sd = lm_state64(m)                    # the oracle sees the bf16-rounded weights
    batch, seqlen = 4, 2048
    ids = _ids(batch, seqlen, cfg.vocab_size, seed=41)
    lengths = (ids != cfg.pad_token_id).sum(dim=1)
    assert lengths.tolist() == [2048, 1748, 2048, 548]
    g = torch.Generator().manual_seed(42)
    # positions: the reference's logits gather (lengths - 1,
    # models/causal_lm.py:110), the last position, and 6 random ones
    pos = torch.cat([(lengths - 1)[:, None], torch.full((batch, 1), seqlen - 1),
                     torch.randint(0, seqlen, (batch, 6), generator=g)], dim=1)
    with torch.no_grad():
        logits = m(ids.to(cuda), lengths.to(cuda), use_cache=True)
        got = torch.gather(logits, 1, pos.to(cuda)[:, :, None].expand(-1, -1, logits.shape[-1]))
        del logits
    print("config4 2 layers: oracle prefill", flush=True)
    extras = {}
    ref, caches = LR.lm_forward(sd, ids, lengths, use_cache=True, logits_at=pos, extras=extras)
    W = sd["lm_head.weight"]
    hmag = _head_mag(extras["hidden"], W)
    assert_close(got, ref, BF16, "c4 prefill logits", hmag, c=C_MODEL, eps=EPS_BF16)
    _check_greedy(got, ref, hmag, "c4 prefill")
    for i, layer in enumerate(m.layers):
        ctx, state = caches[i]
        smag, wmag = extras["state_mag"][i]
        assert_close(layer.ssm._ssm_hiddens, state, BF16, f"c4 layer state {i}", smag, c=C_MODEL,
                     eps=EPS_BF16)
        assert_close(layer.ssm._conv_context, ctx, BF16, f"c4 conv window {i}", wmag, c=C_MODEL,
                     eps=EPS_BF16)
    tokens = torch.randint(1, cfg.vocab_size, (8, batch), generator=g)
    for k in range(8):
        with torch.no_grad():
            got = m.step(tokens[k].to(cuda))
        ex = {}
        ref, caches = LR.lm_step(sd, tokens[k], caches, extras=ex)
        hmag = _head_mag(ex["hidden"], W)
        assert_close(got, ref, BF16, f"c4 step logits {k}", hmag, c=C_MODEL, eps=EPS_BF16)
        _check_greedy(got, ref, hmag, f"c4 step {k}")
    for i, layer in enumerate(m.layers):
        assert_close(layer.ssm._ssm_hiddens, caches[i][1], BF16, f"c4 layer state after steps {i}")
        assert_close(layer.ssm._conv_context, caches[i][0], BF16, f"c4 conv window after steps {i}")


def _snapshot(m):
    return [(l.ssm._conv_context.clone(), l.ssm._ssm_hiddens.clone()) for l in m.layers]


def test_config4_graph_steps_equal_eager_steps(cuda):
    """48 layers: 128 greedy steps replayed from the captured step graph equal
    128 eager steps bit for bit -- the tokens, every layer's state and conv
    window, and the logits of the last step."""
    from ssm_mamba_amd.causal_lm import _greedy_pick
    m, cfg = _model(48, seed=43, dev=cuda)
    batch, seqlen, steps = 4, 2048, 128
    ids = _ids(batch, seqlen, cfg.vocab_size, seed=44).to(cuda)
    lengths = (ids != cfg.pad_token_id).sum(dim=1)
    dec = m.decoder(batch, steps + 1)
    with torch.no_grad():
        dec.capture()
        dec.prefill(ids, lengths)
        dec.replay(steps)
        torch.cuda.synchronize()
        g_tokens = dec.tokens[:, :steps + 1].clone()
        g_state = _snapshot(m)
        g_logits = m.step(dec.token)           # one more step on the graph's caches
        # eager: the same prefill, then `steps` steps launched one by one
        tok = _greedy_pick(m.forward_last(ids, lengths, use_cache=True), 1.0)
        e_tokens = [tok]
        for _ in range(steps):
            tok = _greedy_pick(m.step(tok), 1.0)
            e_tokens.append(tok)
        e_state = _snapshot(m)
        e_logits = m.step(tok)
    assert torch.equal(g_tokens, torch.stack(e_tokens, dim=1)), "graph and eager tokens differ"
    for i, ((gc, gs), (ec, es)) in enumerate(zip(g_state, e_state)):
        assert torch.equal(gs, es), f"layer {i} state differs"
        assert torch.equal(gc, ec), f"layer {i} conv window differs"
    assert torch.equal(g_logits, e_logits)
    print(f"config4 graph == eager: {len(set(g_tokens.flatten().tolist()))} distinct tokens",
          flush=True)


def test_config4_prefill_then_step_equals_longer_prefill(cuda):
    """48 layers: prefill(ids[:, :L]) followed by one step with ids[:, L] gives
    the logits and the per-layer states of prefill(ids[:, :L + 1]) (two
    different kernel paths: the scan and conv kernels against the decode
    step's fused kernels)."""
    m, cfg = _model(48, seed=45, dev=cuda)
    batch, L = 4, 2047
    ids = _ids(batch, L + 1, cfg.vocab_size, seed=46, pads=(0, 0, 0, 0)).to(cuda)
    with torch.no_grad():
        m(ids[:, :L], None, use_cache=True)
        got = m.step(ids[:, L])
        s_state = _snapshot(m)
        logits = m(ids, None, use_cache=True)
        ref = logits[:, L]
        # the LM head's input on the longer prefill's path, for the term sizes
        x = m.embedding(ids).transpose(1, 2).contiguous()
        for layer in m.layers:
            x, _ = layer.forward_cm(x)
        hid = m.norm(x, dim=1)[:, :, L].float()
    mag = _head_mag(hid.cpu(), m.lm_head.weight.float().cpu())
    assert_close(got, ref, BF16, "c4 step vs prefill logits", mag, c=C_MODEL, eps=EPS_BF16)
    for i, layer in enumerate(m.layers):
        assert_close(s_state[i][1], layer.ssm._ssm_hiddens, BF16, f"c4 step vs prefill state {i}")
