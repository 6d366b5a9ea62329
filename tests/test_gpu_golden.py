"""The HIP library, through the C ABI, against the committed golden vectors
(tests/golden/*.npz; fp32 inputs, fp64 expected outputs)."""
import pytest
import torch

from oracle import scan_ref as R
from tests.helpers import Lazy, assert_close
from tests.test_golden import SCANS, UPDATES, load

pytestmark = pytest.mark.gpu


def _dev(g, key, cuda):
    return torch.from_numpy(g[key]).to(cuda) if key in g else None


@pytest.mark.parametrize("path", SCANS, ids=lambda p: p.rsplit("/", 1)[-1])
def test_scan_golden(cuda, path):
    from ssm_mamba_amd import selective_scan as ss
    g = load(path)
    d = {k[3:]: _dev(g, k, cuda) for k in g if k.startswith("in_")}
    pad = "right" if bool(g["padding_right"]) else "left"
    sp = bool(g["softplus"])
    args = (d["u"], d["A"], d["B"], d["C"], d.get("D"), d["delta"], d.get("delta_bias"))
    y = None if d.get("z") is None else torch.empty_like(d["u"])
    out, h = ss.forward(*args, d.get("h_init"), d.get("length"), pad, z=d.get("z"),
                        delta_softplus=sp, out_ungated=y)
    res = ss.backward(*args, h, d.get("h_init"), d["dy"], d.get("dh_last"), d.get("length"), pad,
                      z=d.get("z"), delta_softplus=sp, out_ungated=y)
    torch.cuda.synchronize()
    ref = lambda k: torch.from_numpy(g["out_" + k])
    f32 = torch.float32
    # error-bound magnitudes from the oracle on the fixture's inputs
    c = {k[3:]: torch.from_numpy(g[k]) for k in g if k.startswith("in_")}
    margs = (c["u"], c["delta"], c["A"], c["B"], c["C"], c.get("D"), c.get("delta_bias"),
             c.get("h_init"), c.get("length"), bool(g["padding_right"]), c.get("z"), sp)
    fmag = Lazy(lambda: R.scan_fwd(*margs, magnitude=True))
    bmag = Lazy(lambda: R.scan_bwd(*margs, dy=c["dy"], dh_last=c.get("dh_last"), magnitude=True))
    assert_close(out, ref("y"), f32, "y", fmag.get("y"))
    assert_close(h.permute(0, 3, 1, 2), ref("h_chunks"), f32, "h_chunks", fmag.get("h_chunks"))
    names = ["du", "dA", "dB", "dC", "dD", "ddelta", "ddelta_bias", "dh_init", "dz"]
    for name, val in zip(names, res):
        if ("out_" + name) in g:
            assert_close(val, ref(name), f32, name, bmag.get(name))
        else:
            assert val is None, name


@pytest.mark.parametrize("path", UPDATES, ids=lambda p: p.rsplit("/", 1)[-1])
def test_update_golden(cuda, path):
    from ssm_mamba_amd import selective_update as su
    g = load(path)
    d = {k[3:]: _dev(g, k, cuda) for k in g if k.startswith("in_")}
    keep = d["state"].clone()
    out, new = su.apply_ext(d["x"], d["A"], d["B"], d["C"], d["D"], d["dt"], d["dt_bias"],
                            d["state"], z=d.get("z"), delta_softplus=bool(g["softplus"]))
    torch.cuda.synchronize()
    assert torch.equal(d["state"], keep)
    c = {k[3:]: torch.from_numpy(g[k]) for k in g if k.startswith("in_")}
    mo, mn = R.update(c["state"], c["x"], c["dt"], c["A"], c["B"], c["C"], c.get("D"),
                      c.get("dt_bias"), c.get("z"), bool(g["softplus"]), magnitude=True)
    assert_close(out, torch.from_numpy(g["out_out"]), torch.float32, "out", mo)
    assert_close(new, torch.from_numpy(g["out_state"]), torch.float32, "state", mn)
