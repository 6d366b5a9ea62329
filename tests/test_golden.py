"""The CPU oracle reproduces the committed golden vectors (tests/golden/*.npz,
written by tests/golden/make_golden.py)."""
import glob
import os

import numpy as np
import pytest
import torch

from oracle import scan_ref as R

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SCANS = sorted(glob.glob(os.path.join(HERE, "scan_*.npz")))
UPDATES = sorted(glob.glob(os.path.join(HERE, "update_*.npz")))


def load(path):
    with np.load(path, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def t(arrs, key):
    return torch.from_numpy(arrs[key]) if key in arrs else None


def test_fixtures_present():
    assert len(SCANS) >= 3 and len(UPDATES) >= 2


@pytest.mark.parametrize("path", SCANS, ids=os.path.basename)
def test_oracle_matches_scan_golden(path):
    g = load(path)
    args = [t(g, "in_" + k) for k in ("u", "delta", "A", "B", "C", "D", "delta_bias", "h_init",
                                      "length")]
    pr, sp = bool(g["padding_right"]), bool(g["softplus"])
    z = t(g, "in_z")
    f = R.scan_fwd(*args, pr, z, sp)
    b = R.scan_bwd(*args, pr, z, sp, dy=t(g, "in_dy"), dh_last=t(g, "in_dh_last"))
    got = {"y": f["y"], "h_last": f["h_last"], "h_chunks": f["h_chunks"], **b}
    keys = [k[4:] for k in g if k.startswith("out_")]
    assert {"y", "du", "ddelta", "dA", "dB", "dC"} <= set(keys)
    for k in keys:
        np.testing.assert_allclose(got[k].numpy(), g["out_" + k], rtol=1e-10, atol=1e-12,
                                   err_msg=k)
    for k, inp in (("dD", "D"), ("ddelta_bias", "delta_bias"), ("dh_init", "h_init"), ("dz", "z")):
        # optional gradients are stored exactly when their input is given
        assert (("out_" + k) in g) == (("in_" + inp) in g), k


@pytest.mark.parametrize("path", UPDATES, ids=os.path.basename)
def test_oracle_matches_update_golden(path):
    g = load(path)
    out, new = R.update(*[t(g, "in_" + k) for k in ("state", "x", "dt", "A", "B", "C", "D",
                                                    "dt_bias", "z")],
                        dt_softplus=bool(g["softplus"]))
    np.testing.assert_allclose(out.numpy(), g["out_out"], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(new.numpy(), g["out_state"], rtol=1e-10, atol=1e-12)
