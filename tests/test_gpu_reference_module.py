"""The reference's call sequence through this build's compiled modules, imported
under the reference's top-level names (``import selective_scan``,
``import selective_update``), as the reference's unmodified ``ops/`` files do
(``ops/selective_scan_interface.py:2,45-80``,
``ops/selective_update_interface.py:2,42``):

* forward -> out and the chunk carry h (batch, dim, nchunks, 2*state_dim)
  with nchunks = ceil(seq_len / 128) (``csrc/selective_scan/kernel_config.h:4-10``,
  ``selective_scan.cpp:270-274``);
* h[..., -1, 1::2] is the final state (``ops/selective_scan_interface.py:60``);
* h[..., 0::2] / h[..., 1::2] are the (prod a, state) pairs of every 128-step
  chunk (``csrc/selective_scan/forward_kernel.cu:225-228``);
* the saved h goes back into backward with dout and dh_last, returning the 8
  gradients in the reference's order;
* selective_update.apply is out of place.

Everything is compared with the float64 oracle on the same inputs."""
import importlib
import os
import sys

import pytest
import torch

from oracle import scan_ref as R
from tests.helpers import Lazy, assert_close, make_case, to_dev

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _toplevel(name):
    d = os.path.join(ROOT, "ssm-mamba_amd", "_ext")
    if d not in sys.path:
        sys.path.insert(0, d)
    return importlib.import_module(name)


class RefShapedScanFn(torch.autograd.Function):
    """The reference's SelectiveScanFn call sequence, written against the
    module API: contiguous inputs, forward, save (inputs, h), return
    h[..., -1, 1::2]; backward passes the saved h with dout and dh_last."""

    @staticmethod
    def forward(ctx, u, A, B, C, D, delta, delta_bias, h_init=None, length=None,
                padding_size="left"):
        ss = _toplevel("selective_scan")
        args = [t if t is None else t.contiguous()
                for t in (u, A, B, C, D, delta, delta_bias, h_init, length)]
        out, h = ss.forward(*args, padding_size)
        ctx.save_for_backward(*args[:7], h, args[7], args[8])
        ctx.padding_size = padding_size
        return out, h[..., -1, 1::2]

    @staticmethod
    def backward(ctx, dout, dh_last):
        ss = _toplevel("selective_scan")
        u, A, B, C, D, delta, delta_bias, h, h_init, length = ctx.saved_tensors
        g = ss.backward(u, A, B, C, D, delta, delta_bias, h, h_init, dout.contiguous(),
                        dh_last.contiguous(), length, ctx.padding_size)
        return (*g, None, None)


@pytest.mark.parametrize("padding", ["left", "right"])
@pytest.mark.parametrize("seqlen", [37, 256])
def test_reference_call_sequence(cuda, padding, seqlen):
    batch, dim, nstate = 2, 96, 16
    c = make_case(batch, dim, seqlen, nstate, torch.float32, seed=seqlen, with_z=False,
                  h_init=True)
    d = to_dev(c, cuda)
    length = torch.tensor([seqlen, seqlen - 13])
    names = ("u", "A", "B", "C", "D", "delta", "delta_bias", "h_init")
    leaves = {k: d[k].clone().requires_grad_(True) for k in names}
    out, h_last = RefShapedScanFn.apply(*(leaves[k] for k in names), length.to(cuda), padding)
    g = torch.Generator().manual_seed(seqlen + 1)
    dy = torch.randn(batch, dim, seqlen, generator=g)
    dl = torch.randn(batch, dim, nstate, generator=g)
    ((out * dy.to(cuda)).sum() + (h_last * dl.to(cuda)).sum()).backward()
    pr = padding == "right"
    a = (c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["delta_bias"], c["h_init"], length,
         pr, None, True)
    ref = R.scan_fwd(*a)
    fmag = Lazy(lambda: R.scan_fwd(*a, magnitude=True))
    assert_close(out, ref["y"], torch.float32, "out", fmag.get("y"))
    assert_close(h_last, ref["h_last"], torch.float32, "h_last", fmag.get("h_last"))
    rb = R.scan_bwd(*a, dy=dy, dh_last=dl)
    bmag = Lazy(lambda: R.scan_bwd(*a, dy=dy, dh_last=dl, magnitude=True))
    for k, nm in (("u", "du"), ("A", "dA"), ("B", "dB"), ("C", "dC"), ("D", "dD"),
                  ("delta", "ddelta"), ("delta_bias", "ddelta_bias"), ("h_init", "dh_init")):
        assert_close(leaves[k].grad, rb[nm], torch.float32, nm, bmag.get(nm))


@pytest.mark.parametrize("seqlen,lengths", [(300, (300, 171)), (256, (256, 100)), (100, (100, 71)),
                                            (7, (7, 3))])
def test_chunk_carry_pairs(cuda, seqlen, lengths):
    """h holds (prod a, state) per 128-step chunk, the last chunk's carry the
    final state whether or not 128 divides seq_len; a copy of h (which lacks
    the 16-step states of the view's buffer) is accepted by backward, which
    then recomputes the states, and gives the same gradients bit for bit."""
    ss = _toplevel("selective_scan")
    batch, dim, nstate = 2, 64, 8
    c = make_case(batch, dim, seqlen, nstate, torch.float32, seed=3, with_z=False, h_init=True)
    d = to_dev(c, cuda)
    length = torch.tensor(lengths)
    out, h = ss.forward(d["u"], d["A"], d["B"], d["C"], d["D"], d["delta"], d["delta_bias"],
                        d["h_init"], length.to(cuda), "left")
    K = (seqlen + 127) // 128
    assert h.shape == (batch, dim, K, 2 * nstate)
    a = (c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["delta_bias"], c["h_init"], length,
         False, None, True)
    ref = R.scan_fwd(*a, chunk=128)
    fmag = Lazy(lambda: R.scan_fwd(*a, chunk=128, magnitude=True))
    torch.cuda.synchronize()
    assert_close(h[..., 1::2], ref["h_chunks"], torch.float32, "h_chunks", fmag.get("h_chunks"))
    assert_close(h[..., 0::2], ref["prod_a"], torch.float32, "prod_a")
    assert_close(h[..., -1, 1::2], ref["h_last"], torch.float32, "h_last", fmag.get("h_last"))
    dy = torch.randn(batch, dim, seqlen, generator=torch.Generator().manual_seed(4)).to(cuda)
    dl = torch.zeros(batch, dim, nstate, device=cuda)
    args = (d["u"], d["A"], d["B"], d["C"], d["D"], d["delta"], d["delta_bias"])
    g1 = ss.backward(*args, h, d["h_init"], dy, dl, length.to(cuda), "left")
    g2 = ss.backward(*args, h.contiguous(), d["h_init"], dy, dl, length.to(cuda), "left")
    g3 = ss.backward(*args, h.clone(), d["h_init"], dy, dl, length.to(cuda), "left")
    for x, y, w in zip(g1, g2, g3):
        assert torch.equal(x, y) and torch.equal(x, w)
    rb = R.scan_bwd(*a, dy=dy, dh_last=dl)
    bmag = Lazy(lambda: R.scan_bwd(*a, dy=dy, dh_last=dl, magnitude=True))
    for got, nm in zip(g1, ("du", "dA", "dB", "dC", "dD", "ddelta", "ddelta_bias", "dh_init")):
        assert_close(got, rb[nm], torch.float32, nm, bmag.get(nm))
    with pytest.raises(RuntimeError, match="h must have shape"):
        ss.backward(*args, h[:, :, :, 1:], d["h_init"], dy, dl, length.to(cuda), "left")


def test_toplevel_update_apply(cuda):
    su = _toplevel("selective_update")
    g = torch.Generator().manual_seed(7)
    batch, dim, nstate = 3, 80, 16
    st = torch.randn(batch, dim, nstate, generator=g) * 0.1
    x, dt = torch.randn(batch, dim, generator=g), torch.randn(batch, dim, generator=g)
    Bm, Cm = torch.randn(batch, nstate, generator=g), torch.randn(batch, nstate, generator=g)
    A = -torch.arange(1, nstate + 1, dtype=torch.float32)[None].expand(dim, nstate).contiguous()
    Dv, bias = torch.ones(dim), torch.randn(dim, generator=g) * 0.3 - 2.0
    h = st.to(cuda)
    out, new = su.apply(x.to(cuda), A.to(cuda), Bm.to(cuda), Cm.to(cuda), Dv.to(cuda), dt.to(cuda),
                        bias.to(cuda), h)
    assert new.data_ptr() != h.data_ptr() and torch.equal(h.cpu(), st)
    ro, rn = R.update(st, x, dt, A, Bm, Cm, Dv, bias)
    mo, mn = R.update(st, x, dt, A, Bm, Cm, Dv, bias, magnitude=True)
    assert_close(out, ro, torch.float32, "out", mo)
    assert_close(new, rn, torch.float32, "state", mn)
