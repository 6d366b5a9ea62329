"""Pins the CPU oracle (oracle/scan_ref.py) against what the mathematics fixes.

The reference ships no tests, fixtures or golden vectors and cannot be built
here (CUDA + CUB), so the oracle is pinned by: a brute-force scalar loop,
autograd through an independently written differentiable forward, finite
differences, closed forms (A=0, B=0, u=0), the split-sequence invariant, the
scan == repeated-update invariant and the padding identities.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import scan_ref as R



@pytest.fixture(autouse=True)
def _float64_default():
    """These checks run in float64; the default is restored afterwards so
    other test modules keep float32."""
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def rand_case(batch=2, dim=3, seqlen=37, nstate=4, seed=0, h_init=True, z=True,
              length=None):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    c = {
        "u": r(batch, dim, seqlen),
        "delta": r(batch, dim, seqlen) * 1.5 - 1.0,
        "A": -torch.rand(dim, nstate, generator=g, dtype=torch.float64) * 3 - 0.1,
        "B": r(batch, nstate, seqlen),
        "C": r(batch, nstate, seqlen),
        "D": r(dim),
        "delta_bias": r(dim) * 0.5,
        "h_init": r(batch, dim, nstate) if h_init else None,
        "z": r(batch, dim, seqlen) if z else None,
    }
    return c


def brute_fwd(c, length=None, padding_right=True, delta_softplus=True):
    """Scalar triple loop straight from the recurrence definition."""
    u, dl, A, B, C = c["u"], c["delta"], c["A"], c["B"], c["C"]
    D, bias, h0, z = c["D"], c["delta_bias"], c["h_init"], c["z"]
    batch, dim, L = u.shape
    N = A.shape[1]
    out = torch.zeros(batch, dim, L)
    hl = torch.zeros(batch, dim, N)
    for b in range(batch):
        ln = L if length is None else max(0, min(L, int(length[b])))
        for d in range(dim):
            h = [0.0 if h0 is None else float(h0[b, d, n]) for n in range(N)]
            for t in range(L):
                valid = (t < ln) if padding_right else (t >= L - ln)
                x = float(dl[b, d, t]) + float(bias[d])
                if delta_softplus:
                    x = x if x > 20 else math.log1p(math.exp(x))
                acc = float(D[d]) * float(u[b, d, t])
                for n in range(N):
                    if valid:
                        h[n] = math.exp(x * float(A[d, n])) * h[n] + x * float(u[b, d, t]) * float(B[b, n, t])
                    acc += float(C[b, n, t]) * h[n]
                if z is not None:
                    zz = float(z[b, d, t])
                    acc *= zz / (1.0 + math.exp(-zz))
                out[b, d, t] = acc
            hl[b, d] = torch.tensor(h)
    return out, hl


def naive_fwd_autograd(c, length=None, padding_right=True, delta_softplus=True, gate=True):
    """Differentiable forward written independently of the oracle: per-step
    exp2 form and explicit masking, used only to obtain autograd gradients.
    gate=False returns the output before the z gate."""
    u, dl, A, B, C = c["u"], c["delta"], c["A"], c["B"], c["C"]
    D, bias, h0, z = c["D"], c["delta_bias"], c["h_init"], c["z"]
    batch, dim, L = u.shape
    N = A.shape[1]
    ln = torch.full((batch,), L) if length is None else length.clamp(0, L)
    h = torch.zeros(batch, dim, N) if h0 is None else h0
    outs = []
    for t in range(L):
        if padding_right:
            m = (t < ln).to(u.dtype)
        else:
            m = (t >= L - ln).to(u.dtype)
        m = m[:, None]
        x = dl[:, :, t] + bias[None]
        dt = F.softplus(x, beta=1.0, threshold=20.0) if delta_softplus else x
        dt = dt * m
        a = torch.pow(2.0, (dt[:, :, None] * A[None]) * (1.0 / math.log(2.0)))
        h = a * h + (dt * u[:, :, t])[:, :, None] * B[:, None, :, t]
        y = (h * C[:, None, :, t]).sum(-1) + D[None] * u[:, :, t]
        if z is not None and gate:
            y = y * F.silu(z[:, :, t])
        outs.append(y)
    return torch.stack(outs, -1), h


@pytest.mark.parametrize("padding_right", [True, False])
@pytest.mark.parametrize("use_len", [False, True])
def test_forward_matches_brute_force(padding_right, use_len):
    c = rand_case(batch=2, dim=2, seqlen=19, nstate=3, seed=1)
    length = torch.tensor([19, 7]) if use_len else None
    res = R.scan_fwd(**c, length=length, padding_right=padding_right, chunk=None)
    out, hl = brute_fwd(c, length, padding_right)
    torch.testing.assert_close(res["y"], out, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(res["h_last"], hl, rtol=1e-12, atol=1e-12)


def test_forward_no_softplus_brute_force():
    c = rand_case(batch=1, dim=2, seqlen=11, nstate=2, seed=2)
    c["delta"] = c["delta"].abs() * 0.3  # keep delta > 0 without softplus
    res = R.scan_fwd(**c, delta_softplus=False, chunk=None)
    out, hl = brute_fwd(c, delta_softplus=False)
    torch.testing.assert_close(res["y"], out, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("padding_right", [True, False])
@pytest.mark.parametrize("use_len", [False, True])
@pytest.mark.parametrize("with_z,with_h0", [(True, True), (False, False), (True, False)])
def test_backward_matches_autograd(padding_right, use_len, with_z, with_h0):
    c = rand_case(batch=2, dim=3, seqlen=29, nstate=4, seed=3, h_init=with_h0, z=with_z)
    length = torch.tensor([29, 11]) if use_len else None
    g = torch.Generator().manual_seed(9)
    dy = torch.randn(2, 3, 29, generator=g)
    dlast = torch.randn(2, 3, 4, generator=g)
    leaves = {k: (v.clone().requires_grad_(True) if v is not None else None) for k, v in c.items()}
    # The reference's composition: the scan (whose backward drops the
    # gradient of padded outputs) and then the gate out * silu(z) outside
    # it, which autograd differentiates at every position.
    out, hl = naive_fwd_autograd(leaves, length, padding_right, gate=False)
    mask = R.valid_mask(2, 29, length, padding_right)[:, None, :].to(out.dtype)
    out = out * mask + (out * (1.0 - mask)).detach()
    y = out * F.silu(leaves["z"]) if with_z else out
    loss = (y * dy).sum() + (hl * dlast).sum()
    loss.backward()
    res = R.scan_bwd(**c, length=length, padding_right=padding_right, dy=dy,
                     dh_last=dlast, seg=8)
    pairs = [("du", "u"), ("ddelta", "delta"), ("dA", "A"), ("dB", "B"), ("dC", "C"),
             ("dD", "D"), ("ddelta_bias", "delta_bias")]
    if with_h0:
        pairs.append(("dh_init", "h_init"))
    if with_z:
        pairs.append(("dz", "z"))
    for k, leaf in pairs:
        torch.testing.assert_close(res[k], leaves[leaf].grad, rtol=1e-10, atol=1e-10,
                                   msg=lambda m, k=k: f"{k}: {m}")
    if not with_h0:
        assert res["dh_init"] is None


def test_naive_forward_gradcheck():
    c = rand_case(batch=1, dim=2, seqlen=6, nstate=2, seed=4)
    keys = ["u", "delta", "A", "B", "C", "D", "delta_bias", "h_init", "z"]

    def f(*args):
        cc = dict(zip(keys, args))
        y, h = naive_fwd_autograd(cc)
        return y.sum() + (h * 0.7).sum()

    args = tuple(c[k].clone().requires_grad_(True) for k in keys)
    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-7)


def test_closed_form_A_zero():
    c = rand_case(batch=2, dim=2, seqlen=23, nstate=3, seed=5, z=False)
    c["A"] = torch.zeros_like(c["A"])
    res = R.scan_fwd(**c, chunk=None)
    dt = R.softplus(c["delta"] + c["delta_bias"][None, :, None])
    incr = (dt * c["u"])[:, :, None, :] * c["B"][:, None, :, :]
    h = c["h_init"][..., None] + torch.cumsum(incr, dim=-1)
    out = (h * c["C"][:, None]).sum(2) + c["D"][None, :, None] * c["u"]
    torch.testing.assert_close(res["out"], out, rtol=1e-12, atol=1e-12)


def test_closed_form_B_zero_and_u_zero():
    c = rand_case(batch=2, dim=2, seqlen=17, nstate=3, seed=6, z=False)
    c["B"] = torch.zeros_like(c["B"])
    res = R.scan_fwd(**c, chunk=None)
    dt = R.softplus(c["delta"] + c["delta_bias"][None, :, None])
    decay = torch.exp(torch.cumsum(dt, -1)[:, :, None, :] * c["A"][None, :, :, None])
    h = c["h_init"][..., None] * decay
    out = (h * c["C"][:, None]).sum(2) + c["D"][None, :, None] * c["u"]
    torch.testing.assert_close(res["out"], out, rtol=1e-11, atol=1e-12)
    c2 = rand_case(batch=2, dim=2, seqlen=17, nstate=3, seed=7, h_init=False, z=False)
    c2["u"] = torch.zeros_like(c2["u"])
    r2 = R.scan_fwd(**c2, chunk=None)
    assert r2["out"].abs().max() == 0 and r2["h_last"].abs().max() == 0


def test_split_sequence_invariant():
    c = rand_case(batch=2, dim=3, seqlen=40, nstate=4, seed=8)
    full = R.scan_fwd(**c, chunk=None)
    k = 13
    first = {**c, **{n: c[n][..., :k] for n in ("u", "delta", "B", "C", "z")}}
    second = {**c, **{n: c[n][..., k:] for n in ("u", "delta", "B", "C", "z")}}
    r1 = R.scan_fwd(**first, chunk=None)
    second["h_init"] = r1["h_last"]
    r2 = R.scan_fwd(**second, chunk=None)
    torch.testing.assert_close(torch.cat([r1["y"], r2["y"]], -1), full["y"], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(r2["h_last"], full["h_last"], rtol=1e-12, atol=1e-12)


def test_scan_equals_repeated_update():
    c = rand_case(batch=2, dim=3, seqlen=12, nstate=4, seed=10)
    full = R.scan_fwd(**c, chunk=None)
    h = c["h_init"]
    for t in range(12):
        out, h = R.update(h, c["u"][..., t], c["delta"][..., t], c["A"], c["B"][..., t],
                          c["C"][..., t], c["D"], c["delta_bias"], c["z"][..., t])
        torch.testing.assert_close(out, full["y"][..., t], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(h, full["h_last"], rtol=1e-12, atol=1e-12)


def test_padding_identities():
    c = rand_case(batch=3, dim=2, seqlen=21, nstate=3, seed=11)
    length = torch.tensor([21, 9, 0])
    right = R.scan_fwd(**c, length=length, padding_right=True, chunk=None)
    left = R.scan_fwd(**c, length=length, padding_right=False, chunk=None)
    for b, ln in enumerate(length.tolist()):
        cb = {k: (v[b:b + 1] if (v is not None and k not in ("A", "D", "delta_bias")) else v)
              for k, v in c.items()}
        if ln > 0:
            pre = {**cb, **{n: cb[n][..., :ln] for n in ("u", "delta", "B", "C", "z")}}
            rp = R.scan_fwd(**pre, chunk=None)
            torch.testing.assert_close(right["y"][b:b + 1, :, :ln], rp["y"], rtol=1e-12, atol=1e-12)
            torch.testing.assert_close(right["h_last"][b:b + 1], rp["h_last"], rtol=1e-12, atol=1e-12)
            suf = {**cb, **{n: cb[n][..., 21 - ln:] for n in ("u", "delta", "B", "C", "z")}}
            rs = R.scan_fwd(**suf, chunk=None)
            torch.testing.assert_close(left["y"][b:b + 1, :, 21 - ln:], rs["y"], rtol=1e-12, atol=1e-12)
            torch.testing.assert_close(left["h_last"][b:b + 1], rs["h_last"], rtol=1e-12, atol=1e-12)
        else:
            torch.testing.assert_close(right["h_last"][b], c["h_init"][b])
            torch.testing.assert_close(left["h_last"][b], c["h_init"][b])


def test_h_chunks_are_states_at_chunk_ends():
    c = rand_case(batch=1, dim=2, seqlen=37, nstate=3, seed=12)
    res = R.scan_fwd(**c, chunk=16)
    assert res["h_chunks"].shape == (1, 2, 3, 3)
    for ci, t_end in enumerate([16, 32, 37]):
        pre = {**c, **{n: c[n][..., :t_end] for n in ("u", "delta", "B", "C", "z")}}
        torch.testing.assert_close(res["h_chunks"][:, :, ci], R.scan_fwd(**pre, chunk=None)["h_last"])
    torch.testing.assert_close(res["h_chunks"][:, :, -1], res["h_last"])


def test_softplus_threshold():
    x = torch.tensor([-30.0, -5.0, 0.0, 5.0, 19.999, 20.0, 20.001, 40.0])
    torch.testing.assert_close(R.softplus(x), F.softplus(x, beta=1.0, threshold=20.0))
    xr = x.clone().requires_grad_(True)
    F.softplus(xr, beta=1.0, threshold=20.0).sum().backward()
    torch.testing.assert_close(R.softplus_grad(x), xr.grad)


def test_update_matches_brute_force():
    g = torch.Generator().manual_seed(13)
    B_, D_, N_ = 2, 3, 4
    st = torch.randn(B_, D_, N_, generator=g)
    x, dt, z = (torch.randn(B_, D_, generator=g) for _ in range(3))
    A = -torch.rand(D_, N_, generator=g) * 4
    Bm, Cm = torch.randn(B_, N_, generator=g), torch.randn(B_, N_, generator=g)
    Dv, bias = torch.randn(D_, generator=g), torch.randn(D_, generator=g)
    out, new = R.update(st, x, dt, A, Bm, Cm, Dv, bias, z)
    for b in range(B_):
        for d in range(D_):
            v = float(dt[b, d] + bias[d])
            dl = v if v > 20 else math.log1p(math.exp(v))
            acc = float(Dv[d] * x[b, d])
            for n in range(N_):
                hn = math.exp(dl * float(A[d, n])) * float(st[b, d, n]) + dl * float(x[b, d]) * float(Bm[b, n])
                assert abs(hn - float(new[b, d, n])) < 1e-12
                acc += float(Cm[b, n]) * hn
            zz = float(z[b, d])
            acc *= zz / (1 + math.exp(-zz))
            assert abs(acc - float(out[b, d])) < 1e-12


def test_planted_mistake_is_caught():
    """A wrong-sign decay in a copy of the oracle must fail the brute-force check."""
    c = rand_case(batch=1, dim=2, seqlen=9, nstate=2, seed=14)
    bad = dict(c)
    bad["A"] = -c["A"]
    res = R.scan_fwd(**bad, chunk=None)
    out, _ = brute_fwd(c)
    assert not torch.allclose(res["y"], out, rtol=1e-6, atol=1e-6)


def test_byte_formulas_match_baseline_table():
    f, b = R.algorithmic_bytes_scan(8, 2048, 2048, 16, 2, 2, True)
    assert (f, b) == (270_680_064, 473_202_688)
    f0, _ = R.algorithmic_bytes_scan(2, 1536, 512, 16, 4, 4, True)
    assert f0 == 25_604_096
    f3, b3 = R.algorithmic_bytes_scan(1, 2560, 16384, 16, 4, 4, True)
    assert (f3, b3) == (673_533_952, 1_179_131_904)
    assert R.algorithmic_bytes_update(64, 5120, 16, 2, 2, True) == 44_937_216


def test_prod_a_is_the_running_product_of_decays():
    """prod_a (the first half of the reference's (prod a, h) chunk carry) is the
    product of exp(delta_t A) from t = 0 to each chunk end, padded steps
    counting as 1: checked against a scalar product loop, and through the
    B = 0 closed form h_t = (prod a) h_init."""
    c = rand_case(batch=2, dim=3, seqlen=37, nstate=4, seed=21)
    length = torch.tensor([29, 11])
    for pr in (True, False):
        res = R.scan_fwd(**c, length=length, padding_right=pr, chunk=16)
        pa = res["prod_a"]
        assert pa.shape == (2, 3, 3, 4)
        for b in range(2):
            ln = int(length[b])
            for d in range(3):
                for n in range(4):
                    p = 1.0
                    ends = {15: 0, 31: 1, 36: 2}
                    for t in range(37):
                        valid = (t < ln) if pr else (t >= 37 - ln)
                        if valid:
                            x = float(c["delta"][b, d, t] + c["delta_bias"][d])
                            x = x if x > 20 else math.log1p(math.exp(x))
                            p *= math.exp(x * float(c["A"][d, n]))
                        if t in ends:
                            assert abs(p - float(pa[b, d, ends[t], n])) <= 1e-12 * max(1.0, p)
        zb = {**c, "B": torch.zeros_like(c["B"])}
        r0 = R.scan_fwd(**zb, length=length, padding_right=pr, chunk=16)
        torch.testing.assert_close(r0["h_chunks"], r0["prod_a"] * c["h_init"][:, :, None, :])


def test_magnitude_mode_bounds_and_equals_for_nonnegative_terms():
    """magnitude=True gives sums of |terms|: it bounds |value| everywhere, and it
    equals the value when every term is already non-negative (u, B, C, D,
    h_init, dy, dh_last >= 0, no gate; for the backward also A's sign flipped
    inside the dA / ddelta terms, which the magnitude takes as |A|)."""
    c = rand_case(batch=2, dim=3, seqlen=23, nstate=4, seed=22)
    g = torch.Generator().manual_seed(23)
    dy = torch.randn(2, 3, 23, generator=g, dtype=torch.float64)
    dl = torch.randn(2, 3, 4, generator=g, dtype=torch.float64)
    v = R.scan_fwd(**c)
    m = R.scan_fwd(**c, magnitude=True)
    for k in ("y", "out", "h_chunks", "h_last"):
        assert bool((m[k] >= v[k].abs() * (1 - 1e-12)).all()), k
    vb = R.scan_bwd(**c, dy=dy, dh_last=dl)
    mb = R.scan_bwd(**c, dy=dy, dh_last=dl, magnitude=True)
    for k, x in vb.items():
        if x is not None:
            assert bool((mb[k] >= x.abs() * (1 - 1e-12)).all()), k
    pos = {k: (None if x is None else (x.abs() if k in ("u", "B", "C", "D", "h_init") else x))
           for k, x in c.items()}
    pos["z"] = None
    vp, mp = R.scan_fwd(**pos), R.scan_fwd(**pos, magnitude=True)
    for k in ("y", "h_chunks"):
        torch.testing.assert_close(mp[k], vp[k], rtol=1e-12, atol=0)
    # backward, nonnegative terms: dB, dC, du, dD are sums of products of
    # non-negative factors (the decays keep their sign)
    vbp = R.scan_bwd(**pos, dy=dy.abs(), dh_last=dl.abs())
    mbp = R.scan_bwd(**pos, dy=dy.abs(), dh_last=dl.abs(), magnitude=True)
    for k in ("du", "dB", "dC", "dD", "dh_init"):
        torch.testing.assert_close(mbp[k], vbp[k], rtol=1e-12, atol=0)


def test_error_bound_admits_float32_and_rejects_a_planted_mistake():
    """The float32 oracle stays within error_bound (rtol 1e-4, atol 1e-5, c = 64)
    of the float64 one on every output; a dropped term (the dh_last carry)
    does not."""
    c = R.make_inputs(2, 16, 300, 16, seed=24, with_z=True, h_init=True)
    g = torch.Generator().manual_seed(25)
    dy = torch.randn(2, 16, 300, generator=g)
    dl = torch.randn(2, 16, 16, generator=g)
    args = (c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["delta_bias"], c["h_init"])
    r64 = R.scan_bwd(*args, z=c["z"], dy=dy, dh_last=dl)
    r32 = R.scan_bwd(*args, z=c["z"], dy=dy, dh_last=dl, dtype=torch.float32)
    mag = R.scan_bwd(*args, z=c["z"], dy=dy, dh_last=dl, magnitude=True)
    for k, v in r64.items():
        if v is None:
            continue
        bnd = R.error_bound(v, mag[k], 1e-4, 1e-5, 64.0)
        assert bool(((r32[k].double() - v).abs() <= bnd).all()), k
    bad = R.scan_bwd(*args, z=c["z"], dy=dy, dh_last=None)
    bnd = R.error_bound(r64["dh_init"], mag["dh_init"], 1e-4, 1e-5, 64.0)
    assert not bool(((bad["dh_init"] - r64["dh_init"]).abs() <= bnd).all())
