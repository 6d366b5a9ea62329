"""GPU parity of the HIP selective scan (forward + backward) against the CPU
oracle on the same seeded, dtype-rounded inputs, through the C ABI."""
import pytest
import torch

from oracle import scan_ref as R
from tests.helpers import Lazy, assert_close, make_case, to_dev

pytestmark = pytest.mark.gpu


def _ss():
    from ssm_mamba_amd import selective_scan
    return selective_scan


def oracle_case(c, length, pr, softplus, dy=None, dl=None):
    """The oracle's forward (and backward) on case c, with their magnitude
    runs (sums of |terms|, for the error bound) evaluated lazily."""
    a = (c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["delta_bias"], c["h_init"], length,
         pr, c["z"], softplus)
    ref = R.scan_fwd(*a)
    fmag = Lazy(lambda: R.scan_fwd(*a, magnitude=True))
    if dy is None:
        return ref, fmag, None, None
    rb = R.scan_bwd(*a, dy=dy, dh_last=dl)
    bmag = Lazy(lambda: R.scan_bwd(*a, dy=dy, dh_last=dl, magnitude=True))
    return ref, fmag, rb, bmag


GRAD_NAMES = ["du", "dA", "dB", "dC", "dD", "ddelta", "ddelta_bias", "dh_init"]


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
    print(f"case B={batch} D={dim} L={seqlen} N={nstate} {dtype} seed={seed} pad={padding_side}",
          flush=True)
    out, h = ss.forward(d["u"], d["A"], d["B"], d["C"], d["D"], d["delta"], d["delta_bias"],
                        d["h_init"], ln_dev, padding_side, z=d["z"], delta_softplus=softplus,
                        out_ungated=y)
    if bwd:
        g = torch.Generator().manual_seed(seed + 100)
        dy = torch.randn(batch, dim, seqlen, generator=g).to(dtype)
        dl = torch.randn(batch, dim, nstate, generator=g) if dlast else None
        res = ss.backward(d["u"], d["A"], d["B"], d["C"], d["D"], d["delta"], d["delta_bias"], h,
                          d["h_init"], dy.to(cuda), None if dl is None else dl.to(cuda), ln_dev,
                          padding_side, z=d["z"], delta_softplus=softplus, out_ungated=y)
    else:
        dy = dl = res = None
    torch.cuda.synchronize()
    ref, fmag, rb, bmag = oracle_case(c, length, pr, softplus, dy, dl)
    assert_close(out, ref["y"], dtype, "out", fmag.get("y"))
    if y is not None:
        assert_close(y, ref["out"], dtype, "out_ungated", fmag.get("out"))
    # states are float32 outputs whatever the I/O dtype
    assert_close(h.permute(0, 3, 1, 2), ref["h_chunks"], torch.float32, "h_chunks",
                 fmag.get("h_chunks"))
    if not bwd:
        return
    for nm, got in zip(GRAD_NAMES, res[:8]):
        if rb[nm] is None or got is None:
            assert (nm == "dh_init" and not h_init) or (nm == "dD" and not with_D) or \
                (nm == "ddelta_bias" and not with_bias), nm
            continue
        assert_close(got, rb[nm], dtype, nm, bmag.get(nm))
    if with_z:
        assert_close(res[8], rb["dz"], dtype, "dz", bmag.get("dz"))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_small_aligned(cuda, dtype):
    run_case(cuda, 2, 96, 200, 16, dtype, seed=1, h_init=True, dlast=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("seqlen", [1, 5, 16, 37, 64, 65, 129])
def test_ragged_lengths(cuda, dtype, seqlen):
    run_case(cuda, 1, 70, seqlen, 16, dtype, seed=seqlen, h_init=True, dlast=True)


@pytest.mark.parametrize("nstate", [1, 4, 8, 12, 16, 20, 32, 64, 65, 128, 200, 256])
def test_state_dims(cuda, nstate):
    """Forward and backward for every state-count bucket; past 64 the backward
    runs in chunks of 64 states (the reference accepts state_dim <= 256,
    csrc/selective_scan/selective_scan.cpp:338)."""
    run_case(cuda, 2, 64, 80, nstate, torch.float32, seed=nstate, h_init=True, dlast=True)


@pytest.mark.parametrize("nstate", [128, 256])
def test_state_dims_large_bf16_split(cuda, nstate):
    """Large state counts with bf16 I/O, z, lengths and the sequence split
    (batch 1 x 2 channel blocks, L = 700)."""
    run_case(cuda, 1, 100, 700, nstate, torch.bfloat16, seed=nstate + 1, h_init=True, dlast=True,
             length=torch.tensor([611]), padding_side="left")


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


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch,seqlen", [(2, 200), (1, 264)])
def test_partial_channel_block_aligned(cuda, dtype, batch, seqlen):
    """The aligned path with the last channel block part-filled (80 channels:
    the second block has 16 rows, and three of its four producer waves none)
    and a length that ends inside a 64-step output piece, so the forward's
    four-tile output staging drops the chunks past the end.  Both shapes
    run the sequence split (2 and 3 segments of 128 steps)."""
    run_case(cuda, batch, 80, seqlen, 16, dtype, seed=seqlen + batch, h_init=True, dlast=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("nstate", [1, 5, 12])
def test_sequence_split_few_states(cuda, dtype, nstate):
    """Fewer than 16 states on the role-split path with the sequence split
    (one channel block: 3 segments of L = 300, summaries in 4 parts of 32
    steps, the backward's last parts cut at L or empty): consumer waves and C
    rows past N carry zeros through the summaries and the carries."""
    run_case(cuda, 1, 64, 300, nstate, dtype, seed=50 + nstate, h_init=True, dlast=True,
             length=torch.tensor([283]), padding_side="left")


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
    """Config 1 dtypes and sequence length (bf16 I/O, L=2048) on 256 channels,
    with h_init and dh_last."""
    run_case(cuda, 2, 256, 2048, 16, torch.bfloat16, seed=1, h_init=True, dlast=True)


def test_config1_full(cuda):
    """BASELINE config 1 at full size: B=8, D=2048, N=16, L=2048, bf16 I/O,
    z; every output and gradient (dB / dC reduced over all 2048 channels)
    against the float64 oracle; the backward twice, bit-identical."""
    batch, dim, seqlen, nstate = 8, 2048, 2048, 16
    ss = _ss()
    c = make_case(batch, dim, seqlen, nstate, torch.bfloat16, seed=1)
    d = to_dev(c, cuda)
    y = torch.empty_like(d["u"])
    out, h = ss.forward(d["u"], d["A"], d["B"], d["C"], d["D"], d["delta"], d["delta_bias"],
                        None, None, None, z=d["z"], out_ungated=y)
    dy = torch.randn(batch, dim, seqlen, generator=torch.Generator().manual_seed(5)).bfloat16()
    args = (d["u"], d["A"], d["B"], d["C"], d["D"], d["delta"], d["delta_bias"], h, None,
            dy.to(cuda), None)
    r1 = ss.backward(*args, z=d["z"], out_ungated=y)
    r2 = ss.backward(*args, z=d["z"], out_ungated=y)
    torch.cuda.synchronize()
    for a, b_ in zip(r1, r2):
        if a is not None:
            assert torch.equal(a, b_), "backward is not deterministic"
    ref, fmag, rb, bmag = oracle_case(c, None, True, True, dy, None)
    assert_close(out, ref["y"], torch.bfloat16, "out", fmag.get("y"))
    assert_close(y, ref["out"], torch.bfloat16, "out_ungated", fmag.get("out"))
    assert_close(h.permute(0, 3, 1, 2), ref["h_chunks"], torch.float32, "h_chunks",
                 fmag.get("h_chunks"))
    for nm, got in zip(GRAD_NAMES, r1[:8]):
        if nm != "dh_init":
            assert_close(got, rb[nm], torch.bfloat16, nm, bmag.get(nm))
    assert_close(r1[8], rb["dz"], torch.bfloat16, "dz", bmag.get("dz"))


def test_config3_full(cuda):
    """BASELINE config 3 at full size: B=1, D=2560, N=16, L=16384, fp32,
    delta_raw shifted by +2, z; the sequence-split path (6 segments) with
    every output and gradient against the float64 oracle."""
    run_case(cuda, 1, 2560, 16384, 16, torch.float32, seed=3, delta_shift=2.0)


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
    c["z"] = None
    ref, fmag, rb, bmag = oracle_case(c, length, False, True, dy, dl)
    assert_close(out, ref["y"], dtype, "out", fmag.get("y"))
    assert_close(hl, ref["h_last"], torch.float32, "h_last", fmag.get("h_last"))
    for k, nm in (("u", "du"), ("delta", "ddelta"), ("A", "dA"), ("B", "dB"), ("C", "dC"),
                  ("D", "dD"), ("delta_bias", "ddelta_bias"), ("h_init", "dh_init")):
        assert_close(leaves[k].grad, rb[nm], dtype, nm, bmag.get(nm))


def test_functional_alias(cuda):
    from ssm_mamba_amd.ops import selective_scan_fn
    c = make_case(1, 64, 64, 16, torch.float32, seed=13)
    d = to_dev(c, cuda)
    out, last = selective_scan_fn(d["u"], d["delta"], d["A"], d["B"], d["C"], d["D"], z=d["z"],
                                  delta_bias=d["delta_bias"], return_last_state=True)
    ref, fmag, _, _ = oracle_case(c, None, True, True)
    assert_close(out, ref["y"], torch.float32, "out", fmag.get("y"))
    assert_close(last, ref["h_last"], torch.float32, "h_last", fmag.get("h_last"))


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
    from ssm_mamba_amd.selective_scan import _bc_stride
    outs = []
    for strided in (True, False):
        lu, ld, lz = (t.detach().clone().requires_grad_(True) for t in (u, delta, z))
        if strided:
            # B and C are views of one leaf: the kernels get the batch stride
            Pl = P.detach().clone().requires_grad_(True)
            lB, lC = Pl[:, rank:rank + nstate], Pl[:, rank + nstate:]
            assert bc_batch_strided(lB, lC)
            assert batch == 1 or (_bc_stride(lB) != 0 and not lB.is_contiguous())
        else:
            lB = P[:, rank:rank + nstate].detach().contiguous().requires_grad_(True)
            lC = P[:, rank + nstate:].detach().contiguous().requires_grad_(True)
        yv, last = selective_scan_fn(lu, ld, A, lB, lC, D, z=lz, delta_bias=bias,
                                     return_last_state=True)
        yv.backward(dout)
        if strided:
            dB, dC = Pl.grad[:, rank:rank + nstate], Pl.grad[:, rank + nstate:]
            assert torch.equal(Pl.grad[:, :rank], torch.zeros_like(Pl.grad[:, :rank]))
        else:
            dB, dC = lB.grad, lC.grad
        outs.append([yv.detach(), last.detach(), lu.grad, ld.grad, dB, dC, lz.grad])
    names = ["out", "last", "du", "ddelta", "dB", "dC", "dz"]
    for n, a, b in zip(names, outs[0], outs[1]):
        assert torch.equal(a, b), f"{n} differs between strided and contiguous B/C"
