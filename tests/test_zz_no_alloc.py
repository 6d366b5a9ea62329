"""The allocation-free forward (ssm_selective_scan_fwd_noalloc, static device
scratch) against the workspace forward (ssm_selective_scan_fwd), through the C
ABI: bit-identical outputs on two calls in a row, the second smaller, both
using the scratch (the sequence split's summaries, prepped B/C past 16
states); and shapes whose workspace exceeds the scratch are rejected."""
import pytest
import torch

from tests.helpers import make_case, to_dev

pytestmark = pytest.mark.gpu


def _call(lib, N, noalloc, d, length, pad_right, with_y, pairs):
    batch, dim, seqlen = d["u"].shape
    nstate = d["A"].shape[1]
    dt = N.SSM_BF16 if d["u"].dtype == torch.bfloat16 else N.SSM_F32
    out = torch.full_like(d["u"], float("nan"))
    y = torch.full_like(d["u"], float("nan")) if with_y else None
    # the pair layout: 8 slots of 16 steps per 128-step chunk
    K = 8 * ((seqlen + 127) // 128) if pairs else (seqlen + 15) // 16
    hc = torch.full((batch, K, (2 if pairs else 1) * nstate, dim), float("nan"),
                    device=d["u"].device)
    p = lambda t: None if t is None else t.data_ptr()
    stream = torch.cuda.current_stream().cuda_stream
    args = [batch, dim, seqlen, nstate, dt, p(d["u"]), p(d["delta"]), p(d["A"]), p(d["B"]),
            p(d["C"]), 0, p(d["D"]), p(d["delta_bias"]), p(d["h_init"]), p(length),
            1 if pad_right else 0, p(d["z"]), 1, p(out), p(y), p(hc), 1 if pairs else 0, None]
    if noalloc:
        rc = lib.ssm_selective_scan_fwd_noalloc(*args, stream)
    else:
        wsb = lib.ssm_scan_fwd_workspace_bytes(batch, dim, seqlen, nstate)
        ws = torch.empty(wsb, dtype=torch.uint8, device=d["u"].device)
        rc = lib.ssm_selective_scan_fwd(*args, ws.data_ptr(), wsb, stream)
    N.check(rc)
    torch.cuda.synchronize()
    return out, y, hc


def test_noalloc_forward_equals_workspace_forward(cuda):
    from ssm_mamba_amd import _native as N
    lib = N.lib()
    cases = [
        # (batch, dim, seqlen, nstate, dtype, lengths, pad_right, pairs): the first
        # splits the sequence into 16 segments and preps B/C (32 states)
        (1, 256, 4096, 32, torch.float32, [3001], False, True),
        # smaller second call: bf16, z with the ungated output, 7 segments
        (2, 128, 777, 16, torch.bfloat16, [700, 129], True, False),
    ]
    for i, (batch, dim, seqlen, nstate, dtype, lens, pr, pairs) in enumerate(cases):
        print(f"noalloc case {i}: B={batch} D={dim} L={seqlen} N={nstate} {dtype}", flush=True)
        need = lib.ssm_scan_fwd_workspace_bytes(batch, dim, seqlen, nstate)
        assert 0 < need <= N.SSM_NOALLOC_SCRATCH_BYTES
        d = to_dev(make_case(batch, dim, seqlen, nstate, dtype, seed=50 + i, h_init=True), cuda)
        length = torch.tensor(lens, dtype=torch.int64, device=cuda)
        ref = _call(lib, N, False, d, length, pr, True, pairs)
        got = _call(lib, N, True, d, length, pr, True, pairs)
        for name, a, b in zip(("out", "out_ungated", "h_chunks"), got, ref):
            if a is None:
                assert b is None
                continue
            # bit for bit; NaN where neither call writes (the pair layout's
            # unused decay rows)
            torch.testing.assert_close(a, b, rtol=0, atol=0, equal_nan=True,
                                       msg=f"case {i}: {name} differs from the workspace forward")


def test_noalloc_rejects_shapes_past_the_scratch(cuda):
    from ssm_mamba_amd import _native as N
    lib = N.lib()
    # batch 64 x 2048 channels x 16384 steps x 64 states: the prepped B/C alone
    # is 64 x 32 pairs x 16384 steps x 16 B = 512 MiB
    assert lib.ssm_scan_fwd_workspace_bytes(64, 2048, 16384, 64) > N.SSM_NOALLOC_SCRATCH_BYTES
    # NULL buffers: the size check returns first, and if it ever did not, the
    # forward's own non-NULL checks would reject the call before any launch
    rc = lib.ssm_selective_scan_fwd_noalloc(64, 2048, 16384, 64, N.SSM_F32, None, None, None, None,
                                            None, 0, None, None, None, None, 1, None, 1, None, None,
                                            None, 0, None, None)
    assert rc == 2  # SSM_ERR_UNSUPPORTED
    assert b"static scratch" in lib.ssm_last_error()
