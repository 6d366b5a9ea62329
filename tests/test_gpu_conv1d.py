"""GPU parity of the causal depthwise conv1d (+ SiLU) kernels against the CPU
oracle (oracle/lm_ref.causal_conv, pinned against torch's conv1d), through the
C ABI: forward, and the backward against float64 autograd through the oracle."""
import pytest
import torch
import torch.nn.functional as F

from oracle import lm_ref as LR
from tests.helpers import TOL, assert_close

pytestmark = pytest.mark.gpu


def _case(batch, dim, seqlen, width, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, dim, seqlen, generator=g)
    w = torch.randn(dim, 1, width, generator=g) * 0.5
    b = torch.randn(dim, generator=g) * 0.5
    return x, w, b


def _ref(x, w, b, silu):
    pre = LR.causal_conv(x, w, b)
    return F.silu(pre) if silu else pre


def _wgrad_magnitude(x, w, b, dy, silu):
    """Sums of |terms| of the weight and bias gradients (float64): dweight[c, j]
    = sum_{b,t} dpre * x[t - (k-1) + j] and dbias = sum dpre, dpre = dy *
    act'(pre), taken by their absolute values (the error-bound scale)."""
    xd, wd = x.double(), w.double()
    bd = None if b is None else b.double()
    pre = LR.causal_conv(xd, wd, bd).requires_grad_(True)
    (F.silu(pre) if silu else pre).backward(dy.double())
    dpre = pre.grad.abs()
    wl = wd.clone().requires_grad_(True)
    LR.causal_conv(xd.abs(), wl, None).backward(dpre)
    return wl.grad, dpre.sum((0, 2))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("seqlen", [1, 3, 37, 64, 2048, 2056])
@pytest.mark.parametrize("width", [1, 2, 4, 8])
def test_forward(cuda, dtype, seqlen, width):
    from ssm_mamba_amd.causal_conv1d import causal_conv1d_fn
    x, w, b = _case(2, 5, seqlen, width, seed=seqlen * 10 + width)
    x, w, b = x.to(dtype), w.to(dtype), b.to(dtype)
    for silu in (True, False):
        for bias in (b, None):
            got = causal_conv1d_fn(x.to(cuda), w.to(cuda), None if bias is None else bias.to(cuda),
                                   activation="silu" if silu else None)
            ref = _ref(x.double(), w.double(), None if bias is None else bias.double(), silu)
            assert_close(got, ref, dtype, f"out silu={silu} bias={bias is not None}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("width", [2, 4, 8])
@pytest.mark.parametrize("seqlen", [3, 64, 2051])
def test_forward_window(cuda, dtype, width, seqlen):
    """The decode conv cache written by the forward: the width-1 inputs ending
    at position lengths[b]-1, zero before the row start, lengths clamped to
    [0, seqlen]; without lengths the row's last width-1 inputs.  The output
    is unchanged by the extra write."""
    from ssm_mamba_amd.causal_conv1d import causal_conv1d_fn
    x, w, b = _case(4, 6, seqlen, width, seed=seqlen + width)
    x, w, b = x.to(dtype), w.to(dtype), b.to(dtype)
    lens = torch.tensor([seqlen, 0, 1, seqlen + 5], dtype=torch.long)
    for lengths in (lens, None):
        win = torch.full((4, 6, width - 1), 7.0, dtype=dtype, device=cuda)
        got = causal_conv1d_fn(x.to(cuda), w.to(cuda), b.to(cuda), window=win,
                               lengths=None if lengths is None else lengths.to(cuda))
        assert_close(got, _ref(x.double(), w.double(), b.double(), True), dtype, "out")
        ref = torch.zeros(4, 6, width - 1, dtype=dtype)
        for bb in range(4):
            n = seqlen if lengths is None else min(max(int(lengths[bb]), 0), seqlen)
            for j in range(width - 1):
                t = n - (width - 1) + j
                if t >= 0:
                    ref[bb, :, j] = x[bb, :, t]
        assert torch.equal(win.cpu(), ref), f"window lengths={lengths}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("seqlen", [5, 40, 2048, 4099])
@pytest.mark.parametrize("width", [1, 3, 4, 8])
def test_backward(cuda, dtype, seqlen, width):
    from ssm_mamba_amd.causal_conv1d import causal_conv1d_fn
    x, w, b = _case(3, 4, seqlen, width, seed=seqlen + width)
    x, w, b = x.to(dtype), w.to(dtype), b.to(dtype)
    dy = torch.randn(3, 4, seqlen, generator=torch.Generator().manual_seed(7)).to(dtype)
    xg, wg, bg = (t.to(cuda).requires_grad_(True) for t in (x, w, b))
    causal_conv1d_fn(xg, wg, bg, activation="silu").backward(dy.to(cuda))
    xr, wr, br = (t.double().requires_grad_(True) for t in (x, w, b))
    _ref(xr, wr, br, True).backward(dy.double())
    assert_close(xg.grad, xr.grad, dtype, "dx")
    # weight / bias gradients are sums over batch x seqlen terms
    mw, mb = _wgrad_magnitude(x, w, b, dy, True)
    assert_close(wg.grad, wr.grad, dtype, "dweight", mw)
    assert_close(bg.grad, br.grad, dtype, "dbias", mb)


def test_backward_without_bias_or_activation(cuda):
    from ssm_mamba_amd.causal_conv1d import causal_conv1d_fn
    x, w, _ = _case(2, 6, 96, 4, seed=3)
    dy = torch.randn(2, 6, 96, generator=torch.Generator().manual_seed(8))
    xg, wg = x.to(cuda).requires_grad_(True), w.to(cuda).requires_grad_(True)
    causal_conv1d_fn(xg, wg, None, activation=None).backward(dy.to(cuda))
    xr, wr = x.double().requires_grad_(True), w.double().requires_grad_(True)
    _ref(xr, wr, None, False).backward(dy.double())
    assert_close(xg.grad, xr.grad, torch.float32, "dx")
    mw, _ = _wgrad_magnitude(x, w, None, dy, False)
    assert_close(wg.grad, wr.grad, torch.float32, "dweight", mw)


def test_deterministic_and_rejects_bad_width(cuda):
    from ssm_mamba_amd.causal_conv1d import causal_conv1d_fn
    x, w, b = _case(4, 64, 512, 4, seed=9)
    dy = torch.randn(4, 64, 512)
    grads = []
    for _ in range(2):
        wg = w.to(cuda).requires_grad_(True)
        causal_conv1d_fn(x.to(cuda), wg, b.to(cuda)).backward(dy.to(cuda))
        grads.append(wg.grad.clone())
    assert torch.equal(grads[0], grads[1])
    with pytest.raises(RuntimeError, match="width"):
        causal_conv1d_fn(x.to(cuda), torch.randn(64, 1, 9, device=cuda), None)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("seqlen", [37, 2048])
def test_forward_batch_strided(cuda, dtype, seqlen):
    """x as a channel slice of a larger activation (the x half of the
    in-projection output): read in place through its batch stride, the same
    bits as from a contiguous copy, window and lengths included."""
    from ssm_mamba_amd.causal_conv1d import causal_conv1d_fn
    x, w, b = _case(3, 2 * 40, seqlen, 4, seed=seqlen)
    big = x.to(dtype).to(cuda)
    xs = big[:, 8:48]                       # batch stride 80 * seqlen, offset 8 rows
    assert not xs.is_contiguous() and xs.stride(0) == 80 * seqlen
    wd, bd = w[:40].to(dtype).to(cuda), b[:40].to(dtype).to(cuda)
    lens = torch.tensor([seqlen, 5, 0], dtype=torch.long, device=cuda)
    win_a = torch.zeros(3, 40, 3, dtype=dtype, device=cuda)
    win_b = torch.zeros_like(win_a)
    got = causal_conv1d_fn(xs, wd, bd, window=win_a, lengths=lens)
    ref = causal_conv1d_fn(xs.contiguous(), wd, bd, window=win_b, lengths=lens)
    assert torch.equal(got, ref) and torch.equal(win_a, win_b)
    assert_close(got, _ref(x[:, 8:48].to(dtype).double(), w[:40].to(dtype).double(),
                           b[:40].to(dtype).double(), True), dtype, "out strided")


def test_backward_batch_strided_input(cuda):
    """Autograd through a batch-strided x (a channel slice): the gradients
    equal those of a contiguous copy bit for bit."""
    from ssm_mamba_amd.causal_conv1d import causal_conv1d_fn
    x, w, b = _case(2, 64, 96, 4, seed=77)
    big = x.repeat(1, 2, 1).to(cuda)                 # (2, 128, 96); use channels 32..95
    dy = torch.randn(2, 64, 96, generator=torch.Generator().manual_seed(78)).to(cuda)
    grads = []
    for strided in (True, False):
        xb = big.clone().requires_grad_(True)
        xs = xb[:, 32:96] if strided else xb[:, 32:96].contiguous()
        wd = w.to(cuda).requires_grad_(True)
        bd = b.to(cuda).requires_grad_(True)
        causal_conv1d_fn(xs, wd, bd).backward(dy)
        grads.append((xb.grad.clone(), wd.grad.clone(), bd.grad.clone()))
    for g1, g2 in zip(*grads):
        assert torch.equal(g1, g2)
