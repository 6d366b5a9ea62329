"""GPU parity of the HIP decode step (selective_state_update) against the CPU
oracle, through the C ABI."""
import math

import pytest
import torch

from oracle import scan_ref as R
from tests.helpers import TOL, assert_close, make_case, to_dev

pytestmark = pytest.mark.gpu


def step_inputs(batch, dim, nstate, dtype, seed, with_z=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, dim, generator=g).to(dtype)
    dt = torch.randn(batch, dim, generator=g).to(dtype)
    z = torch.randn(batch, dim, generator=g).to(dtype) if with_z else None
    B = torch.randn(batch, nstate, generator=g).to(dtype)
    C = torch.randn(batch, nstate, generator=g).to(dtype)
    return x, dt, z, B, C


def params(dim, nstate, seed=0):
    g = torch.Generator().manual_seed(seed)
    A = -torch.arange(1, nstate + 1, dtype=torch.float32)[None].expand(dim, nstate).contiguous()
    dtv = torch.exp(torch.rand(dim, generator=g) * (math.log(0.1) - math.log(1e-3))
                    + math.log(1e-3)).clamp(min=1e-4)
    return A, torch.ones(dim), R.inv_softplus(dtv)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("nstate", [1, 3, 4, 12, 16, 32, 64, 200, 256])
def test_step_shapes(cuda, dtype, nstate):
    from ssm_mamba_amd import selective_update as su
    batch, dim = 3, 70
    A, D, bias = params(dim, nstate, seed=nstate)
    g = torch.Generator().manual_seed(1)
    st = torch.randn(batch, dim, nstate, generator=g) * 0.1
    x, dt, z, B, C = step_inputs(batch, dim, nstate, dtype, seed=nstate)
    dev = lambda t: None if t is None else t.to(cuda)
    out, new = su.apply_ext(dev(x), dev(A), dev(B), dev(C), dev(D), dev(dt), dev(bias), dev(st), z=dev(z))
    ro, rn = R.update(st, x, dt, A, B, C, D, bias, z)
    mo, mn = R.update(st, x, dt, A, B, C, D, bias, z, magnitude=True)
    assert_close(out, ro, dtype, "out", mo)
    assert_close(new, rn, torch.float32, "state", mn)


def test_no_softplus_no_z_inplace(cuda):
    from ssm_mamba_amd import selective_update as su
    batch, dim, nstate = 2, 64, 16
    A, D, bias = params(dim, nstate)
    st = torch.randn(batch, dim, nstate) * 0.1
    x, dt, _, B, C = step_inputs(batch, dim, nstate, torch.float32, seed=5, with_z=False)
    dt = dt.abs() * 0.1
    h = st.clone().to(cuda)
    out, new = su.apply_ext(x.to(cuda), A.to(cuda), B.to(cuda), C.to(cuda), None, dt.to(cuda), None,
                            h, delta_softplus=False, inplace=True)
    assert new.data_ptr() == h.data_ptr()
    ro, rn = R.update(st, x, dt, A, B, C, None, None, None, dt_softplus=False)
    mo, mn = R.update(st, x, dt, A, B, C, None, None, None, dt_softplus=False, magnitude=True)
    assert_close(out, ro, torch.float32, "out", mo)
    assert_close(h, rn, torch.float32, "state", mn)


def test_reference_api_out_of_place(cuda):
    from ssm_mamba_amd.ops import SelectiveUpdateFn
    batch, dim, nstate = 4, 128, 16
    A, D, bias = params(dim, nstate)
    st = (torch.randn(batch, dim, nstate) * 0.1).to(cuda)
    keep = st.clone()
    x, dt, _, B, C = step_inputs(batch, dim, nstate, torch.float32, seed=6, with_z=False)
    out, new = SelectiveUpdateFn.apply(x.to(cuda), A.to(cuda), B.to(cuda), C.to(cuda), D.to(cuda),
                                       dt.to(cuda), bias.to(cuda), st)
    assert torch.equal(st, keep), "SelectiveUpdateFn must not modify its input state"
    ro, rn = R.update(keep.cpu(), x, dt, A, B, C, D, bias, None)
    mo, mn = R.update(keep.cpu(), x, dt, A, B, C, D, bias, None, magnitude=True)
    assert_close(out, ro, torch.float32, "out", mo)
    assert_close(new, rn, torch.float32, "state", mn)


def test_config2_stepwise(cuda):
    """B=64, D=5120, N=16; fp32 state ~ 0.1 N(0,1); bf16
    x/dt/z/B/C; the GPU and CPU chains evolve independently and are compared
    at every one of the 256 steps.  The state's error bound uses the sum of
    the absolute values of its terms, carried along the chain by the oracle
    (the magnitude recurrence over all earlier steps)."""
    from ssm_mamba_amd.ops import selective_state_update
    batch, dim, nstate = 64, 5120, 16
    A, D, bias = params(dim, nstate, seed=2)
    g = torch.Generator().manual_seed(2)
    st = torch.randn(batch, dim, nstate, generator=g) * 0.1
    ref_state = st.double()
    mag_state = st.double().abs()
    gpu_state = st.to(cuda)
    Ad, Dd, bd = A.to(cuda), D.to(cuda), bias.to(cuda)
    for k in range(256):
        x, dt, z, B, C = step_inputs(batch, dim, nstate, torch.bfloat16, seed=1000 + k)
        out = selective_state_update(gpu_state, x.to(cuda), dt.to(cuda), Ad, B.to(cuda), C.to(cuda),
                                     Dd, z.to(cuda), bd)
        ro, ref_state = R.update(ref_state, x, dt, A, B, C, D, bias, z)
        mo, mag_state = R.update(mag_state, x, dt, A, B, C, D, bias, z, magnitude=True)
        assert_close(out, ro, torch.bfloat16, f"out step {k}", mo)
        assert_close(gpu_state, ref_state, torch.float32, f"state step {k}", mag_state)


def test_scan_equals_update_loop_on_gpu(cuda):
    """scan over L steps == L decode steps (both on the GPU)."""
    from ssm_mamba_amd import selective_scan as ss
    from ssm_mamba_amd import selective_update as su
    c = to_dev(make_case(2, 64, 24, 16, torch.float32, seed=14, h_init=True), cuda)
    out, h = ss.forward(c["u"], c["A"], c["B"], c["C"], c["D"], c["delta"], c["delta_bias"],
                        c["h_init"], None, None, z=c["z"])
    st = c["h_init"].clone()
    for t in range(24):
        o, st = su.apply_ext(c["u"][..., t].contiguous(), c["A"], c["B"][..., t].contiguous(),
                             c["C"][..., t].contiguous(), c["D"], c["delta"][..., t].contiguous(),
                             c["delta_bias"], st, z=c["z"][..., t].contiguous())
        torch.testing.assert_close(o, out[..., t], **TOL[torch.float32])
    torch.testing.assert_close(st, ss.last_state(h), rtol=1e-4, atol=1e-5)
