"""Writes the golden vectors under tests/golden/ from the CPU oracle
(oracle/scan_ref.py, float64).

The reference ships no tests or fixtures, and its CUDA implementation cannot
be built here.  The oracle is pinned in tests/test_oracle.py against brute
force, autograd, finite differences and closed forms.  These files freeze its
outputs on small cases that cover the path's edges:

* right and left padding, including a zero length;
* h_init, dh_last and the z gate;
* no softplus, no D and no bias;
* an odd state count and the decode step.

The CPU suite checks that the oracle still reproduces them; the GPU suite
checks the HIP library against them.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import scan_ref as R  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

# name: (batch, dim, seqlen, nstate, seed, lengths, padding_right, h_init, z, softplus, D, bias, dh_last)
SCAN_CASES = {
    "scan_right_pad": (2, 6, 37, 4, 11, [37, 23], True, True, True, True, True, True, True),
    "scan_left_pad": (2, 5, 33, 3, 12, [30, 0], False, False, False, True, True, True, False),
    "scan_plain_odd": (1, 7, 16, 5, 13, None, True, True, True, False, False, False, True),
}
# name: (batch, dim, nstate, seed, z, softplus)
UPDATE_CASES = {
    "update_z": (3, 5, 6, 21, True, True),
    "update_nosp": (2, 4, 3, 22, False, False),
}


def _f32(t):
    return t.to(torch.float32)


def make_scan(name, batch, dim, seqlen, nstate, seed, lengths, pad_right, with_h0, with_z,
              softplus, with_D, with_bias, with_dlast):
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, dtype=torch.float32)
    u = rn(batch, dim, seqlen)
    delta = rn(batch, dim, seqlen) * 0.8 - 0.5
    if not softplus:
        delta = delta.abs() * 0.3 + 0.01
    A = -(torch.rand(dim, nstate, generator=g) * 2.0 + 0.2)
    B = rn(batch, nstate, seqlen)
    C = rn(batch, nstate, seqlen)
    D = rn(dim) if with_D else None
    bias = rn(dim) * 0.5 if with_bias else None
    h0 = rn(batch, dim, nstate) * 0.5 if with_h0 else None
    z = rn(batch, dim, seqlen) if with_z else None
    ln = None if lengths is None else torch.tensor(lengths, dtype=torch.int64)
    dy = rn(batch, dim, seqlen)
    dlast = rn(batch, dim, nstate) if with_dlast else None
    f = R.scan_fwd(u, delta, A, B, C, D, bias, h0, ln, pad_right, z, softplus)
    b = R.scan_bwd(u, delta, A, B, C, D, bias, h0, ln, pad_right, z, softplus, dy=dy, dh_last=dlast)
    arrs = {"padding_right": np.array(int(pad_right)), "softplus": np.array(int(softplus))}
    ins = dict(u=u, delta=delta, A=A, B=B, C=C, D=D, delta_bias=bias, h_init=h0, z=z, dy=dy,
               dh_last=dlast)
    for k, v in ins.items():
        if v is not None:
            arrs["in_" + k] = _f32(v).numpy()
    if ln is not None:
        arrs["in_length"] = ln.numpy()
    for k in ("y", "h_last", "h_chunks"):
        arrs["out_" + k] = f[k].numpy()
    present = {"dD": with_D, "ddelta_bias": with_bias, "dh_init": with_h0, "dz": with_z}
    for k in ("du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dh_init", "dz"):
        if present.get(k, True):
            arrs["out_" + k] = b[k].numpy()
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrs)


def make_update(name, batch, dim, nstate, seed, with_z, softplus):
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, dtype=torch.float32)
    st = rn(batch, dim, nstate) * 0.3
    x = rn(batch, dim)
    dt = rn(batch, dim) if softplus else rn(batch, dim).abs() * 0.2
    A = -(torch.rand(dim, nstate, generator=g) * 2.0 + 0.2)
    B = rn(batch, nstate)
    C = rn(batch, nstate)
    D = rn(dim)
    bias = rn(dim) * 0.5
    z = rn(batch, dim) if with_z else None
    out, new = R.update(st, x, dt, A, B, C, D, bias, z, dt_softplus=softplus)
    arrs = {"softplus": np.array(int(softplus))}
    for k, v in dict(state=st, x=x, dt=dt, A=A, B=B, C=C, D=D, dt_bias=bias, z=z).items():
        if v is not None:
            arrs["in_" + k] = _f32(v).numpy()
    arrs["out_out"] = out.numpy()
    arrs["out_state"] = new.numpy()
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrs)


def main():
    for name, args in SCAN_CASES.items():
        make_scan(name, *args)
    for name, args in UPDATE_CASES.items():
        make_update(name, *args)
    print("wrote", ", ".join(list(SCAN_CASES) + list(UPDATE_CASES)))


if __name__ == "__main__":
    main()
