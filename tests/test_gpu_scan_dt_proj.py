"""GPU parity of the selective-scan forward with the fused step-size
projection (ssm_selective_scan_fwd_dt_proj), through the C ABI.

The inputs are those of a Mamba block at the scan (modules/mamba.py:141-171):
the token-major x-projection output ssm_params (batch, L, R + 2N) with each
token's row [dt | B | C], the step-size weight W_dt (dim, R), u, z, A, D,
delta_bias.  Two checks pin the result:

* delta_raw, returned in delta_out, against float64 W_dt @ dt^T: one bf16
  rounding (2^-8 relative) plus the float32 rounding of a sum of R products,
  c * 2^-24 * sum|terms|;
* out and the last state against the float64 oracle run on exactly those
  delta_raw values, with B and C taken from the token rows, at the bounds of
  the scan's own parity tests.

A third check runs the same call without delta_out and requires the same bits
(the store is a side output only)."""
import pytest
import torch

from oracle import scan_ref as R
from ssm_mamba_amd import _native as N
from tests.helpers import EPS_BF16, Lazy, assert_close, make_case

pytestmark = pytest.mark.gpu

TOL_DELTA = dict(rtol=EPS_BF16, atol=0.0)


def run_dt_case(cuda, batch, dim, seqlen, nstate, rank, seed, with_z=True, h_init=False,
                length=None, padding_side="left", pstride_pad=0, z_strided=False):
    print(f"dt_proj case B={batch} D={dim} L={seqlen} N={nstate} R={rank} seed={seed} "
          f"z={with_z} h0={h_init} len={None if length is None else length.tolist()} "
          f"pad={padding_side} pstride+{pstride_pad}", flush=True)
    lib = N.lib()
    assert lib.ssm_selective_scan_fwd_dt_proj_supported(batch, dim, seqlen, nstate, rank,
                                                         N.SSM_BF16) == 1
    c = make_case(batch, dim, seqlen, nstate, torch.bfloat16, seed=seed, with_z=with_z,
                  h_init=h_init)
    g = torch.Generator().manual_seed(seed + 7)
    dt = (torch.randn(batch, seqlen, rank, generator=g) * 0.5).to(torch.bfloat16)
    # W_dt as the reference initialises it: uniform in +-rank^-0.5 (modules/mamba.py:52-60)
    w = ((torch.rand(dim, rank, generator=g) * 2 - 1) * rank ** -0.5).to(torch.bfloat16)
    P = rank + 2 * nstate
    rows = torch.cat([dt, c["B"].transpose(1, 2), c["C"].transpose(1, 2)], dim=2)  # (b, L, P)
    pstride = seqlen * P + pstride_pad
    buf = torch.zeros(batch * pstride, dtype=torch.bfloat16)
    for b in range(batch):
        buf[b * pstride:b * pstride + seqlen * P] = rows[b].reshape(-1)
    dev = lambda t: None if t is None else t.to(cuda).contiguous()
    u, z, A, Dv, bias, h0 = (dev(c[k]) for k in ("u", "z", "A", "D", "delta_bias", "h_init"))
    zbs = 0
    if z_strided and z is not None:
        # z as the gate half of a (batch, 2 dim, L) in-projection output
        zz = torch.empty(batch, 2 * dim, seqlen, dtype=z.dtype, device=cuda).normal_()
        zz[:, dim:] = z
        z, zbs = zz[:, dim:], 2 * dim * seqlen
    params, wd = dev(buf), dev(w)
    ln = None if length is None else length.to(cuda)
    out = torch.full((batch, dim, seqlen), float("nan"), dtype=torch.bfloat16, device=cuda)
    dout = torch.full_like(out, float("nan"))
    last = torch.full((batch, dim, nstate), float("nan"), device=cuda)
    ws = torch.empty(lib.ssm_scan_fwd_workspace_bytes(batch, dim, seqlen, nstate),
                     dtype=torch.uint8, device=cuda)
    ptr = lambda t: None if t is None else t.data_ptr()
    pr = 1 if padding_side == "right" else 0
    stream = torch.cuda.current_stream().cuda_stream

    def call(delta_out, o, hl):
        N.check(lib.ssm_selective_scan_fwd_dt_proj(
            batch, dim, seqlen, nstate, rank, N.SSM_BF16, u.data_ptr(), params.data_ptr(),
            pstride, wd.data_ptr(), A.data_ptr(), Dv.data_ptr(), bias.data_ptr(), ptr(h0), ptr(ln),
            pr, ptr(z), zbs, 1, o.data_ptr(), ptr(delta_out), hl.data_ptr(), ws.data_ptr(), ws.numel(),
            stream))

    call(dout, out, last)
    out2, last2 = torch.empty_like(out), torch.empty_like(last)
    call(None, out2, last2)
    torch.cuda.synchronize()
    # delta_raw against float64 W_dt @ dt^T
    wdd, dtd = w.double(), dt.double()
    d_ref = torch.einsum("dr,blr->bdl", wdd, dtd)
    assert_close(dout, d_ref, torch.bfloat16, "delta_raw", tol=TOL_DELTA,
                 mag=lambda: torch.einsum("dr,blr->bdl", wdd.abs(), dtd.abs()))
    # the scan on those step sizes against the oracle
    a = (c["u"], dout.cpu(), c["A"], c["B"], c["C"], c["D"], c["delta_bias"], c["h_init"], length,
         pr == 1, c["z"], True)
    ref = R.scan_fwd(*a)
    mag = Lazy(lambda: R.scan_fwd(*a, magnitude=True))
    assert_close(out, ref["y"], torch.bfloat16, "out", mag.get("y"))
    assert_close(last, ref["h_last"], torch.float32, "h_last", mag.get("h_last"))
    assert torch.equal(out, out2) and torch.equal(last, last2), "delta_out changed the result"


@pytest.mark.parametrize("seqlen", [16, 64, 200, 2048])
def test_dt_proj_aligned(cuda, seqlen):
    run_dt_case(cuda, 2, 128, seqlen, 16, 64, seed=seqlen)


@pytest.mark.parametrize("seqlen", [1, 5, 37, 130, 515])
def test_dt_proj_ragged(cuda, seqlen):
    """Lengths that are not multiples of 8 (the pointer path), one channel
    block part-filled."""
    run_dt_case(cuda, 1, 80, seqlen, 16, 64, seed=100 + seqlen)


@pytest.mark.parametrize("rank,nstate", [(8, 4), (16, 8), (40, 12), (48, 16), (56, 16)])
def test_dt_proj_ranks(cuda, rank, nstate):
    """Ranks below 64 leave rank groups of the MFMA operands empty (zero
    weights); fewer than 16 states leave B/C columns unused."""
    run_dt_case(cuda, 2, 64, 96, nstate, rank, seed=rank * 10 + nstate)


def test_dt_proj_state_and_lengths(cuda):
    """h_init, left-padded lengths (0, partial, full), the gate."""
    run_dt_case(cuda, 3, 130, 300, 16, 64, seed=5, h_init=True,
                length=torch.tensor([0, 123, 300], dtype=torch.int64))


def test_dt_proj_right_padding_no_gate(cuda):
    run_dt_case(cuda, 2, 64, 96, 16, 32, seed=6, with_z=False, padding_side="right",
                length=torch.tensor([50, 96], dtype=torch.int64))


def test_dt_proj_batch_stride(cuda):
    """Batch rows of ssm_params further apart than seqlen * P (a padded or
    sliced buffer)."""
    run_dt_case(cuda, 2, 64, 64, 16, 64, seed=8, pstride_pad=24)


def test_dt_proj_gate_batch_stride(cuda):
    """z read in place as the gate half of the in-projection output, aligned
    and ragged lengths."""
    run_dt_case(cuda, 3, 128, 256, 16, 64, seed=11, z_strided=True)
    run_dt_case(cuda, 2, 64, 37, 16, 64, seed=12, z_strided=True,
                length=torch.tensor([37, 20], dtype=torch.int64))


def test_dt_proj_sequence_split(cuda):
    """Few batch rows x channel blocks: the sequence is split into segments
    with the segment summaries, which run the projection too."""
    run_dt_case(cuda, 1, 64, 4096, 16, 64, seed=9, h_init=True)


def test_dt_proj_config4_layer(cuda):
    """A config-4 layer's scan: batch 4, d_inner 2048, L 2048, N 16, rank 64."""
    run_dt_case(cuda, 4, 2048, 2048, 16, 64, seed=10)


def test_dt_proj_rejects_unsupported(cuda):
    lib = N.lib()
    assert lib.ssm_selective_scan_fwd_dt_proj_supported(2, 64, 64, 16, 64, N.SSM_F32) == 0
    assert lib.ssm_selective_scan_fwd_dt_proj_supported(2, 64, 64, 16, 72, N.SSM_BF16) == 0
    assert lib.ssm_selective_scan_fwd_dt_proj_supported(2, 64, 64, 16, 60, N.SSM_BF16) == 0
    assert lib.ssm_selective_scan_fwd_dt_proj_supported(2, 64, 64, 32, 64, N.SSM_BF16) == 0
    assert lib.ssm_selective_scan_fwd_dt_proj_supported(2, 64, 64, 6, 64, N.SSM_BF16) == 0


def _sweep_config(seed):
    import random
    g = random.Random(seed)
    batch = g.choice([1, 2, 3])
    seqlen = g.choice([1, 2, 7, 16, 33, 64, 100, 128, 250, 256, 300, 513, 600])
    length = None
    if g.random() < 0.5:
        length = torch.tensor([g.randint(0, seqlen) for _ in range(batch)], dtype=torch.int64)
    return dict(batch=batch, dim=g.choice([64, 80, 130, 256]), seqlen=seqlen,
                nstate=g.choice([4, 8, 12, 16, 16]), rank=g.choice([8, 16, 24, 32, 40, 48, 56, 64]),
                with_z=g.random() < 0.8, h_init=g.random() < 0.5, length=length,
                padding_side=g.choice(["left", "right"]), pstride_pad=g.choice([0, 0, 8, 40]),
                z_strided=g.random() < 0.3)


@pytest.mark.parametrize("seed", range(40))
def test_dt_proj_sweep(cuda, seed):
    """Seeded irregular shapes: part-filled channel blocks, ragged and aligned
    lengths, 4-16 states, ranks 8-64, gate or none, h_init, lengths on either
    side, padded ssm_params rows and a batch-strided gate."""
    c = _sweep_config(500 + seed)
    run_dt_case(cuda, c["batch"], c["dim"], c["seqlen"], c["nstate"], c["rank"], seed=900 + seed,
                with_z=c["with_z"], h_init=c["h_init"], length=c["length"],
                padding_side=c["padding_side"], pstride_pad=c["pstride_pad"],
                z_strided=c["z_strided"])
