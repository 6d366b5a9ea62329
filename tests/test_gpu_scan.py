"""GPU parity of the HIP selective scan (forward + backward) against the CPU
oracle on the same seeded, dtype-rounded inputs, through the C ABI."""
import pytest
import torch

from oracle import scan_ref as R
from tests.helpers import assert_close, make_case, to_dev

pytestmark = pytest.mark.gpu


def _ss():
    from ssm_mamba_amd import selective_scan
    return selective_scan


def run_case(cuda, batch, dim, seqlen, nstate, dtype, *, seed=0, with_z=True, h_init=False,
             length=None, padding_side="right", softplus=True, dlast=False, delta_shift=0.0,
             bwd=True, with_D=True, with_bias=True, positive_delta=False):
    ss = _ss()
    c = make_case(batch, dim, seqlen, nstate, dtype, seed=seed, with_z=with_z, h_init=h_init,
                  delta_shift=delta_shift)
    if positive_delta:  # without softplus the step size is delta itself and must stay > 0
        c["delta"] = (c["delta"].float().abs() * 0.2).to(dtype)
    if not with_D:
        c["D"] = None
    if not with_bias:
        c["delta_bias"] = None
    d = to_dev(c, cuda)
    ln_dev = None if length is None else length.to(cuda)
    pr = (padding_side or "right") == "right"
    y = None if d["z"] is None else torch.empty_like(d["u"])
    out, h = ss.forward(d["u"], d["A"], d["B"], d["C"], d["D"], d["delta"], d["delta_bias"],
                        d["h_init"], ln_dev, padding_side, z=d["z"], delta_softplus=softplus,
                        out_ungated=y)
    ref = R.scan_fwd(c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["delta_bias"],
                     c["h_init"], length, pr, c["z"], softplus)
    torch.cuda.synchronize()
    assert_close(out, ref["y"], dtype, "out")
    if y is not None:
        assert_close(y, ref["out"], dtype, "out_ungated")
    assert_close(h.permute(0, 3, 1, 2), ref["h_chunks"],
                 torch.float32 if dtype == torch.float32 else dtype, "h_chunks", scale_atol=True)
    if not bwd:
        return
    g = torch.Generator().manual_seed(seed + 100)
    dy = torch.randn(batch, dim, seqlen, generator=g).to(dtype)
    dl = torch.randn(batch, dim, nstate, generator=g) if dlast else None
    res = ss.backward(d["u"], d["A"], d["B"], d["C"], d["D"], d["delta"], d["delta_bias"], h,
                      d["h_init"], dy.to(cuda), None if dl is None else dl.to(cuda), ln_dev,
                      padding_side, z=d["z"], delta_softplus=softplus, out_ungated=y)
    rb = R.scan_bwd(c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["delta_bias"],
                    c["h_init"], length, pr, c["z"], softplus, dy=dy, dh_last=dl)
    torch.cuda.synchronize()
    names = ["du", "dA", "dB", "dC", "dD", "ddelta", "ddelta_bias", "dh_init"]
    for nm, got in zip(names, res[:8]):
        if rb[nm] is None or got is None:
            assert (nm == "dh_init" and not h_init) or (nm == "dD" and not with_D) or \
                (nm == "ddelta_bias" and not with_bias), nm
            continue
        assert_close(got, rb[nm], dtype, nm, scale_atol=nm in ("dA", "dB", "dC", "dD", "ddelta_bias"))
    if with_z:
        assert_close(res[8], rb["dz"], dtype, "dz")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_small_aligned(cuda, dtype):
    run_case(cuda, 2, 96, 200, 16, dtype, seed=1, h_init=True, dlast=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("seqlen", [1, 5, 16, 37, 64, 65, 129])
def test_ragged_lengths(cuda, dtype, seqlen):
    run_case(cuda, 1, 70, seqlen, 16, dtype, seed=seqlen, h_init=True, dlast=True)


@pytest.mark.parametrize("nstate", [1, 4, 8, 12, 16, 20, 32, 64])
def test_state_dims(cuda, nstate):
    run_case(cuda, 2, 64, 80, nstate, torch.float32, seed=nstate, h_init=True, dlast=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("nstate", [1, 3])
def test_odd_partial_count(cuda, dtype, nstate):
    """batch * nstate * seqlen not a multiple of 4: the dB/dC partial sums
    take the element-wise reduction path."""
    run_case(cuda, 1, 64, 37, nstate, dtype, seed=40 + nstate, h_init=True, dlast=True)


@pytest.mark.parametrize("nstate", [128, 200, 256])
def test_state_dims_forward_large(cuda, nstate):
    run_case(cuda, 1, 64, 48, nstate, torch.float32, seed=nstate, bwd=False)


@pytest.mark.parametrize("padding_side", ["right", "left"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lengths(cuda, padding_side, dtype):
    length = torch.tensor([150, 0, 1, 200], dtype=torch.int64)
    run_case(cuda, 4, 64, 200, 16, dtype, seed=7, length=length, padding_side=padding_side,
             h_init=True, dlast=True)


@pytest.mark.parametrize("padding_side,lengths", [("right", [300, 777]), ("left", [1, 650]),
                                                   ("right", [0, 129])])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sequence_split_many_segments(cuda, padding_side, lengths, dtype):
    """Batch 2 x 2 channel blocks fills 4 workgroups, so the scan splits L = 777
    into 7 segments (6 of 128 steps and a ragged tail); lengths start and end
    inside segments; h_init, dh_last and z carry across every boundary."""
    run_case(cuda, 2, 80, 777, 16, dtype, seed=11, length=torch.tensor(lengths),
             padding_side=padding_side, h_init=True, dlast=True)


@pytest.mark.parametrize("nstate", [32, 64])
def test_sequence_split_state_groups(cuda, nstate):
    """More than 16 states take the summaries' multi-group path."""
    run_case(cuda, 1, 64, 500, nstate, torch.float32, seed=nstate + 3, h_init=True, dlast=True,
             length=torch.tensor([431]), padding_side="left")


def test_sequence_split_forward_large_state(cuda):
    run_case(cuda, 1, 64, 300, 200, torch.float32, seed=5, h_init=True, bwd=False)


def test_no_softplus_no_z_no_D(cuda):
    run_case(cuda, 2, 64, 96, 16, torch.float32, seed=8, with_z=False, softplus=False,
             with_D=False, with_bias=False, positive_delta=True)


def test_config0(cuda):
    """B=2, D=1536, N=16, L=512, fp32, z."""
    run_case(cuda, 2, 1536, 512, 16, torch.float32, seed=0)


def test_config1_reduced_channels(cuda):
    """Config 1 dtypes and sequence length (bf16 I/O, L=2048) on 256 channels."""
    run_case(cuda, 2, 256, 2048, 16, torch.bfloat16, seed=1)


def test_config3_reduced_channels(cuda):
    """Config 3 (fp32, L=16384, delta shifted by +2) on 64 channels."""
    run_case(cuda, 1, 64, 16384, 16, torch.float32, seed=3, delta_shift=2.0)


def test_config1_full_size_properties(cuda):
    """Full config-1 size: forward on a channel subset against the oracle,
    bitwise determinism, and dB/dC additivity over channel halves."""
    ss = _ss()
    batch, dim, seqlen, nstate = 8, 2048, 2048, 16
    c = make_case(batch, dim, seqlen, nstate, torch.bfloat16, seed=1)
    d = to_dev(c, cuda)
    y = torch.empty_like(d["u"])
    out, h = ss.forward(d["u"], d["A"], d["B"], d["C"], d["D"], d["delta"], d["delta_bias"],
                        None, None, None, z=d["z"], out_ungated=y)
    sub = slice(0, 2048, 97)  # 22 channels spread over the channel blocks
    cs = {k: (v[:, sub] if k in ("u", "delta", "z") else v) for k, v in c.items()}
    cs["A"], cs["D"], cs["delta_bias"] = c["A"][sub], c["D"][sub], c["delta_bias"][sub]
    ref = R.scan_fwd(cs["u"], cs["delta"], cs["A"], cs["B"], cs["C"], cs["D"], cs["delta_bias"],
                     None, None, True, cs["z"], True, dtype=torch.float64)
    assert_close(out[:, sub], ref["y"], torch.bfloat16, "out[subset]")
    assert_close(h.permute(0, 3, 1, 2)[:, sub], ref["h_chunks"], torch.bfloat16, "h[subset]",
                 scale_atol=True)
    g = torch.Generator().manual_seed(5)
    dy = torch.randn(batch, dim, seqlen, generator=g).to(torch.bfloat16).to(cuda)
    args = (d["u"], d["A"], d["B"], d["C"], d["D"], d["delta"], d["delta_bias"], h, None, dy, None)
    r1 = ss.backward(*args, z=d["z"], out_ungated=y)
    r2 = ss.backward(*args, z=d["z"], out_ungated=y)
    for a, b_ in zip(r1, r2):
        if a is not None:
            assert torch.equal(a, b_), "backward is not deterministic"
    # dB over all channels == sum of dB over two channel halves (fp32 partials)
    halves = []
    for lo, hi in ((0, 1024), (1024, 2048)):
        dh = {k: (v[:, lo:hi].contiguous() if k in ("u", "delta", "z") else v) for k, v in d.items()}
        dh["A"], dh["D"], dh["delta_bias"] = d["A"][lo:hi].contiguous(), d["D"][lo:hi].contiguous(), \
            d["delta_bias"][lo:hi].contiguous()
        yh = torch.empty_like(dh["u"])
        _, hh = ss.forward(dh["u"], dh["A"], dh["B"], dh["C"], dh["D"], dh["delta"],
                           dh["delta_bias"], None, None, None, z=dh["z"], out_ungated=yh)
        halves.append(ss.backward(dh["u"], dh["A"], dh["B"], dh["C"], dh["D"], dh["delta"],
                                  dh["delta_bias"], hh, None, dy[:, lo:hi].contiguous(), None,
                                  z=dh["z"], out_ungated=yh))
    for idx, nm in ((2, "dB"), (3, "dC")):
        # each of the three results is rounded to bf16 once (relative error
        # <= 2^-9); the fp32 partial sums agree to ~1e-6
        h0, h1, full = halves[0][idx].float(), halves[1][idx].float(), r1[idx].float()
        bound = 2.0 ** -8 * (h0.abs() + h1.abs() + full.abs()) + 1e-5
        err = (full - (h0 + h1)).abs()
        assert bool((err <= bound).all()), f"{nm} additivity: max excess {(err - bound).max().item():.3g}"
    # per-channel gradients of the subset against the oracle
    rb = R.scan_bwd(cs["u"], cs["delta"], cs["A"], cs["B"], cs["C"], cs["D"], cs["delta_bias"],
                    None, None, True, cs["z"], True, dy=dy.cpu()[:, sub], dh_last=None)
    assert_close(r1[0][:, sub], rb["du"], torch.bfloat16, "du[subset]")
    assert_close(r1[5][:, sub], rb["ddelta"], torch.bfloat16, "ddelta[subset]")
    assert_close(r1[8][:, sub], rb["dz"], torch.bfloat16, "dz[subset]")
    assert_close(r1[1][sub], rb["dA"], torch.bfloat16, "dA[subset]", scale_atol=True)
    assert_close(r1[4][sub], rb["dD"], torch.bfloat16, "dD[subset]", scale_atol=True)
    assert_close(r1[6][sub], rb["ddelta_bias"], torch.bfloat16, "dbias[subset]", scale_atol=True)


def test_split_sequence_on_gpu(cuda):
    """scan(x) == scan(x[:k]) then scan(x[k:], h_init=h_last), on the GPU."""
    ss = _ss()
    c = to_dev(make_case(2, 128, 256, 16, torch.float32, seed=9), cuda)
    out, h = ss.forward(c["u"], c["A"], c["B"], c["C"], c["D"], c["delta"], c["delta_bias"],
                        None, None, None, z=c["z"])
    k = 96
    p1 = {n: c[n][..., :k].contiguous() for n in ("u", "delta", "B", "C", "z")}
    p2 = {n: c[n][..., k:].contiguous() for n in ("u", "delta", "B", "C", "z")}
    o1, h1 = ss.forward(p1["u"], c["A"], p1["B"], p1["C"], c["D"], p1["delta"], c["delta_bias"],
                        None, None, None, z=p1["z"])
    o2, h2 = ss.forward(p2["u"], c["A"], p2["B"], p2["C"], c["D"], p2["delta"], c["delta_bias"],
                        ss.last_state(h1).contiguous(), None, None, z=p2["z"])
    torch.testing.assert_close(torch.cat([o1, o2], -1), out, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(ss.last_state(h2), ss.last_state(h), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_reference_api_autograd(cuda, dtype):
    """SelectiveScanFn (the reference's class and argument order) through autograd."""
    from ssm_mamba_amd.ops import SelectiveScanFn
    batch, dim, seqlen, nstate = 2, 64, 100, 16
    c = make_case(batch, dim, seqlen, nstate, dtype, seed=11, with_z=False, h_init=True)
    d = to_dev(c, cuda)
    leaves = {k: d[k].clone().requires_grad_(True)
              for k in ("u", "A", "B", "C", "D", "delta", "delta_bias", "h_init")}
    length = torch.tensor([100, 60])
    out, hl = SelectiveScanFn.apply(leaves["u"], leaves["A"], leaves["B"], leaves["C"],
                                    leaves["D"], leaves["delta"], leaves["delta_bias"],
                                    leaves["h_init"], length.to(cuda))
    g = torch.Generator().manual_seed(12)
    dy = torch.randn(batch, dim, seqlen, generator=g).to(dtype)
    dl = torch.randn(batch, dim, nstate, generator=g)
    ((out.float() * dy.to(cuda).float()).sum() + (hl * dl.to(cuda)).sum()).backward()
    # the reference's default padding is "left" (ops/selective_scan_interface.py:20)
    ref = R.scan_fwd(c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["delta_bias"],
                     c["h_init"], length, False, None, True)
    assert_close(out, ref["y"], dtype, "out")
    assert_close(hl, ref["h_last"], dtype, "h_last", scale_atol=True)
    rb = R.scan_bwd(c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["delta_bias"],
                    c["h_init"], length, False, None, True, dy=dy, dh_last=dl)
    for k, nm in (("u", "du"), ("delta", "ddelta"), ("A", "dA"), ("B", "dB"), ("C", "dC"),
                  ("D", "dD"), ("delta_bias", "ddelta_bias"), ("h_init", "dh_init")):
        assert_close(leaves[k].grad, rb[nm], dtype, nm, scale_atol=nm in ("dA", "dB", "dC", "dD", "ddelta_bias"))


def test_functional_alias(cuda):
    from ssm_mamba_amd.ops import selective_scan_fn
    c = make_case(1, 64, 64, 16, torch.float32, seed=13)
    d = to_dev(c, cuda)
    out, last = selective_scan_fn(d["u"], d["delta"], d["A"], d["B"], d["C"], d["D"], z=d["z"],
                                  delta_bias=d["delta_bias"], return_last_state=True)
    ref = R.scan_fwd(c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["delta_bias"], None,
                     None, True, c["z"], True)
    assert_close(out, ref["y"], torch.float32, "out")
    assert_close(last, ref["h_last"], torch.float32, "last", scale_atol=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch,dim,seqlen,nstate", [
    (2, 64, 300, 16),     # split path (few workgroups), partial last tile
    (4, 512, 256, 16),    # one segment per row
    (3, 128, 64, 5),      # odd state count
    (1, 64, 48, 16),      # batch 1 (the stride is never used)
])
def test_batch_strided_bc(cuda, dtype, batch, dim, seqlen, nstate):
    """B and C passed as channel slices of one larger activation (the
    x-projection output of the model): rows contiguous, one batch stride
    larger than nstate * seqlen.  Forward and backward must equal the
    contiguous copies bit for bit (the kernels read the same values)."""
    from ssm_mamba_amd.ops import selective_scan_fn
    from ssm_mamba_amd.selective_scan import bc_batch_strided
    g = torch.Generator().manual_seed(batch * 1000 + dim + seqlen + nstate)
    rank = 8
    P = torch.randn(batch, rank + 2 * nstate, seqlen, generator=g).to(dtype).to(cuda)
    u = torch.randn(batch, dim, seqlen, generator=g).to(dtype).to(cuda)
    delta = (0.5 * torch.randn(batch, dim, seqlen, generator=g)).to(dtype).to(cuda)
    z = torch.randn(batch, dim, seqlen, generator=g).to(dtype).to(cuda)
    A = (-torch.rand(dim, nstate, generator=g) - 0.5).to(cuda)
    D = torch.randn(dim, generator=g).to(cuda)
    bias = (0.3 * torch.randn(dim, generator=g)).to(cuda)
    dout = torch.randn(batch, dim, seqlen, generator=g).to(dtype).to(cuda)
    Bv, Cv = P[:, rank:rank + nstate], P[:, rank + nstate:]
    assert bc_batch_strided(Bv, Cv) and (batch == 1 or not Bv.is_contiguous())
    outs = []
    for B, C in ((Bv, Cv), (Bv.contiguous(), Cv.contiguous())):
        leaves = [t.detach().clone().requires_grad_(True) for t in (u, delta, B, C, z)]
        lu, ld, lB, lC, lz = leaves
        y, last = selective_scan_fn(lu, ld, A, lB, lC, D, z=lz, delta_bias=bias,
                                    return_last_state=True)
        y.backward(dout)
        outs.append([y.detach(), last.detach()] + [t.grad for t in leaves])
    names = ["out", "last", "du", "ddelta", "dB", "dC", "dz"]
    for n, a, b in zip(names, outs[0], outs[1]):
        assert torch.equal(a, b), f"{n} differs between strided and contiguous B/C"
