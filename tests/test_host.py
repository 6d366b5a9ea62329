"""CPU-side checks of the host layer: the C ABI library loads and exports every
symbol declared in include/ssm_mamba.h (no compute calls), workspace/chunk
queries, and the reference-mirroring validation errors."""
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    txt = open(os.path.join(ROOT, "include", "ssm_mamba.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(ssm_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_header_symbols():
    from ssm_mamba_amd import _native as N
    lib = N.lib()
    names = header_functions()
    assert len(names) >= 7
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/ssm_mamba.h but not exported"
        assert n in N.SIGNATURES, f"{n} has no ctypes signature"


def test_queries():
    from ssm_mamba_amd import _native as N
    lib = N.lib()
    assert lib.ssm_abi_version() == N.ABI_VERSION
    assert [lib.ssm_scan_nchunks(x) for x in (0, 1, 16, 17, 2048)] == [0, 1, 1, 2, 128]
    # the reference's kernel_config::get_num_chunks (128-step chunks)
    assert [lib.ssm_scan_ref_nchunks(x) for x in (0, 1, 128, 129, 2048)] == [0, 1, 1, 2, 16]
    # fwd workspace: prepped B/C, fp32, rows padded to 16 steps, states padded to 4
    # prepped B/C (batch x pairs x padded steps x 4 floats) + a 256-byte store sink
    assert lib.ssm_scan_fwd_workspace_bytes(8, 2048, 2048, 16) == 8 * 4 * 2048 * 8 * 4 + 256
    # pairs padded to a multiple of 8: 8 pairs x 16 steps x 4 floats, + the sink
    assert lib.ssm_scan_fwd_workspace_bytes(1, 64, 5, 3) == 8 * 16 * 4 * 4 + 256
    assert lib.ssm_scan_bwd_workspace_bytes(8, 2048, 2048, 16) > 2 * 32 * 8 * 16 * 2048 * 4


def test_invalid_arguments_return_errors():
    """The C ABI rejects bad sizes before touching any pointer (no GPU needed)."""
    from ssm_mamba_amd import _native as N
    lib = N.lib()
    rc = lib.ssm_selective_scan_fwd(1, 1, 1, 300, 0, *([None] * 5), 0,
                                    *([None] * 4), 1, None, 1, None, None, None, 0, None, None,
                                    0, None)
    assert rc == 2 and b"state_dim <= 256" in lib.ssm_last_error()
    rc = lib.ssm_selective_scan_fwd(1, 1, 0, 16, 0, *([None] * 5), 0,
                                    *([None] * 4), 1, None, 1, None, None, None, 0, None, None,
                                    0, None)
    assert rc == 1 and b">= 1" in lib.ssm_last_error()
    rc = lib.ssm_selective_scan_fwd(1, 1, 1, 16, 7, *([None] * 5), 0,
                                    *([None] * 4), 1, None, 1, None, None, None, 0, None, None,
                                    0, None)
    assert rc == 1 and b"dtype" in lib.ssm_last_error()
    rc = lib.ssm_selective_scan_fwd(1, 1, 1, 16, 0, *([None] * 5), 0,
                                    *([None] * 4), 1, None, 1, None, None, None, 0, None, None,
                                    0, None)
    assert rc == 1 and b"non-NULL" in lib.ssm_last_error()
    rc = lib.ssm_selective_scan_bwd(1, 1, 1, 257, 0, *([None] * 5), 0, *([None] * 4), 1, None, None, 1, None, 0,
                                    None, None, *([None] * 9), None, 0, None)
    assert rc == 2 and b"state_dim <= 256" in lib.ssm_last_error()
    # past 64 states the backward runs in chunks: its workspace holds the
    # chunks' per-position sums (2 x chunks x batch x dim x seqlen fp32)
    w64 = lib.ssm_scan_bwd_workspace_bytes(2, 64, 80, 64)
    w65 = lib.ssm_scan_bwd_workspace_bytes(2, 64, 80, 65)
    assert w65 - w64 >= 2 * 2 * 2 * 64 * 80 * 4
    rc = lib.ssm_selective_state_update(1, 1, 16, 0, *([None] * 10), 1, None, None)
    assert rc == 1 and b"non-NULL" in lib.ssm_last_error()


def test_gate_arguments_are_checked():
    """With z the backward needs the forward's ungated output and dz; without z
    neither may be given.  The checks return before any pointer is used, so
    placeholder addresses stand in for the device buffers (no GPU needed)."""
    from ssm_mamba_amd import _native as N
    lib = N.lib()
    P = 4096  # never dereferenced: every call below fails its argument checks

    def bwd(z, y, dz):
        return lib.ssm_selective_scan_bwd(1, 64, 16, 16, 0, P, P, P, P, P, 0, None, None, None, None,
                                          1, z, y, 1, P, 0, P, None, P, P, P, P, P, None, None, None,
                                          dz, P, 1 << 30, None)

    for z, y, dz in ((P, None, P), (P, P, None), (P, None, None)):
        assert bwd(z, y, dz) == 1 and b"requires dz and out_ungated" in lib.ssm_last_error()
    for y, dz in ((P, None), (None, P), (P, P)):
        assert bwd(None, y, dz) == 1 and b"require z" in lib.ssm_last_error()
    rc = lib.ssm_selective_scan_fwd(1, 64, 16, 16, 0, P, P, P, P, P, 0, None, None, None, None, 1,
                                    None, 1, P, P, P, 0, None, P, 1 << 30, None)
    assert rc == 1 and b"out_ungated requires z" in lib.ssm_last_error()
    rc = lib.ssm_selective_scan_fwd(1, 64, 16, 16, 0, P, P, P, P, P, 0, None, None, None, None, 1,
                                    None, 1, P, None, None, 1, None, P, 1 << 30, None)
    assert rc == 1 and b"h_pairs requires h_chunks" in lib.ssm_last_error()


def test_folded_xproj_queries_and_checks():
    """The folded x-projection: its block count (16 channels per block,
    params_dim <= 256) and the argument checks of the two calls that carry it,
    which return before any pointer is used (no GPU needed)."""
    from ssm_mamba_amd import _native as N
    lib = N.lib()
    blocks = lib.ssm_decode_xproj_blocks
    assert blocks(2048, 96) == 128 and blocks(16, 3) == 1 and blocks(2048, 256) == 128
    assert blocks(24, 96) == 0 and blocks(2048, 257) == 0 and blocks(0, 96) == 0
    assert blocks(2048, 0) == 0
    P = 4096  # never dereferenced

    def in_proj(dim, wx, nout, part):
        return lib.ssm_decode_in_proj_conv(4, dim, 1024, 4, N.SSM_BF16, P, P, P, 1e-6, None, P,
                                           None, P, P, P, wx, nout, part, None)

    assert in_proj(2048, P, 96, None) == 1 and b"go together" in lib.ssm_last_error()
    assert in_proj(2048, None, 96, P) == 1 and b"go together" in lib.ssm_last_error()
    assert in_proj(24, P, 96, P) == 2 and b"folded x-projection" in lib.ssm_last_error()
    assert in_proj(2048, P, 300, P) == 2 and b"folded x-projection" in lib.ssm_last_error()

    def step(blocks_arg):
        return lib.ssm_decode_ssm_step(4, 2048, 16, 64, N.SSM_BF16, P, blocks_arg, P, None, P,
                                       None, P, P, 4096, P, P, None)

    for b in (5, 127, -1):
        assert step(b) == 1 and b"params_blocks must be 0 or" in lib.ssm_last_error()


def test_bc_batch_stride_is_checked():
    """A B/C batch stride below nstate * seqlen is rejected (0 means contiguous)."""
    from ssm_mamba_amd import _native as N
    lib = N.lib()
    P = 4096  # never dereferenced
    ws = 1 << 30
    rc = lib.ssm_selective_scan_fwd(2, 64, 16, 16, 0, P, P, P, P, P, 16 * 16 - 8, None, None, None,
                                    None, 1, None, 1, P, None, P, 0, None, P, ws, None)
    assert rc == 1 and b"bc_batch_stride" in lib.ssm_last_error()
    rc = lib.ssm_selective_scan_bwd(2, 64, 16, 16, 0, P, P, P, P, P, 100, None, None, None, None,
                                    1, None, None, 1, P, 0, P, None, P, P, P, P, P, None, None, None,
                                    None, P, ws, None)
    assert rc == 1 and b"bc_batch_stride" in lib.ssm_last_error()


def test_dt_proj_shapes_and_arguments_are_checked():
    """The fused step-size projection's shape query and argument checks run on
    the host (fake addresses are never dereferenced: every call here returns
    before any launch)."""
    from ssm_mamba_amd import _native as N
    lib = N.lib()
    ok = lambda *a: lib.ssm_selective_scan_fwd_dt_proj_supported(*a)
    assert ok(4, 2048, 2048, 16, 64, N.SSM_BF16) == 1
    assert ok(1, 80, 37, 4, 8, N.SSM_BF16) == 1
    assert ok(4, 2048, 2048, 16, 64, N.SSM_F32) == 0      # bf16 only
    assert ok(4, 2048, 2048, 16, 72, N.SSM_BF16) == 0     # rank > 64
    assert ok(4, 2048, 2048, 16, 60, N.SSM_BF16) == 0     # rank not a multiple of 8
    assert ok(4, 2048, 2048, 32, 64, N.SSM_BF16) == 0     # N > 16
    assert ok(4, 2048, 2048, 6, 64, N.SSM_BF16) == 0      # N not a multiple of 4
    assert ok(1, 64, 1 << 24, 16, 64, N.SSM_BF16) == 0    # token rows past 2^31 bytes
    P = 4096  # a 16-byte aligned fake address
    ws = 1 << 30

    def call(**kw):
        a = dict(batch=2, dim=64, seqlen=16, nstate=16, rank=64, dtype=N.SSM_BF16, u=P, params=P,
                 pstride=0, w=P, A=P, z=None, zbs=0, out=P, ws=P)
        a.update(kw)
        return lib.ssm_selective_scan_fwd_dt_proj(
            a["batch"], a["dim"], a["seqlen"], a["nstate"], a["rank"], a["dtype"], a["u"],
            a["params"], a["pstride"], a["w"], a["A"], None, None, None, None, 0, a["z"], a["zbs"],
            1, a["out"], None, None, a["ws"], ws, None)

    # SSM_ERR_INVALID = 1, SSM_ERR_UNSUPPORTED = 2
    assert call(dtype=N.SSM_F32) == 2 and b"bf16" in lib.ssm_last_error()
    assert call(rank=0) == 1 and b"dt_rank" in lib.ssm_last_error()
    assert call(params=None) == 1 and b"non-NULL" in lib.ssm_last_error()
    assert call(pstride=16 * 96 - 8) == 1 and b"params_batch_stride" in lib.ssm_last_error()
    assert call(pstride=16 * 96 + 4) == 2 and b"16-byte" in lib.ssm_last_error()
    assert call(params=P + 8) == 2 and b"16-byte" in lib.ssm_last_error()
    assert call(z=P, zbs=64 * 16 - 8) == 1 and b"z_batch_stride" in lib.ssm_last_error()
    assert call(ws=None) == 1 and b"workspace" in lib.ssm_last_error()
    # the shape query leaves the last error message alone
    assert ok(2, 64, 16, 16, 72, N.SSM_BF16) == 0 and b"workspace" in lib.ssm_last_error()


def test_conv_batch_stride_is_checked():
    """The conv forward's x batch stride: 0 (contiguous) or at least dim * seqlen."""
    from ssm_mamba_amd import _native as N
    lib = N.lib()
    P = 4096  # never dereferenced
    rc = lib.ssm_causal_conv1d_fwd(2, 8, 16, 4, N.SSM_BF16, P, 8 * 16 - 1, P, None, 1, P, None,
                                   None, None)
    assert rc == 1 and b"x_batch_stride" in lib.ssm_last_error()


def _scan_args(batch=2, dim=4, seqlen=8, nstate=3):
    return dict(u=torch.randn(batch, dim, seqlen), A=torch.randn(dim, nstate),
                B=torch.randn(batch, nstate, seqlen), C=torch.randn(batch, nstate, seqlen),
                D=torch.randn(dim), delta=torch.randn(batch, dim, seqlen), delta_bias=torch.randn(dim))


@pytest.mark.parametrize("mutate,msg", [
    (lambda a: a.update(u=a["u"][0]), "u must be a 3D tensor"),
    (lambda a: a.update(A=a["A"][0]), "A must be a 2D tensor"),
    (lambda a: a.update(A=torch.randn(4, 300)), "state_dim <= 256"),
    (lambda a: None, "u must be a CUDA tensor"),
])
def test_scan_validation_messages(mutate, msg):
    """Validation mirrors csrc/selective_scan/selective_scan.cpp:15-32,229-268."""
    from ssm_mamba_amd import selective_scan as ss
    a = _scan_args()
    mutate(a)
    with pytest.raises(RuntimeError, match=msg):
        ss.forward(a["u"], a["A"], a["B"], a["C"], a["D"], a["delta"], a["delta_bias"])


def test_update_device_check():
    """The reference never checks the device of selective_update's inputs
    (selective_update.cpp:11-21); this build does."""
    from ssm_mamba_amd import selective_update as su
    with pytest.raises(RuntimeError, match="u must be a CUDA tensor"):
        su.apply(torch.randn(2, 4), torch.randn(4, 3), torch.randn(2, 3), torch.randn(2, 3),
                 torch.randn(4), torch.randn(2, 4), torch.randn(4), torch.randn(2, 4, 3))


def test_product_path_has_no_oracle_import():
    """The package never imports the oracle (test infrastructure only)."""
    pkg = os.path.join(ROOT, "ssm-mamba_amd")
    for dp, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(dp, f)).read()
                assert "import oracle" not in src and "from oracle" not in src, f


def _toplevel(name):
    """The extension module under the reference's top-level name (its
    directory on sys.path, as the reference's ops/ files import it)."""
    import importlib
    import sys
    d = os.path.join(ROOT, "ssm-mamba_amd", "_ext")
    if d not in sys.path:
        sys.path.insert(0, d)
    return importlib.import_module(name)


def test_extension_modules_mirror_the_reference_bindings():
    """selective_scan.{forward, backward} and selective_update.apply exist under
    the reference's module names with its parameter order
    (csrc/selective_scan/bindings.cpp:5-8, csrc/selective_update/bindings.cpp:5-7,
    csrc/selective_scan/selective_scan.h:73-99, selective_update.h:32-41)."""
    ss, su = _toplevel("selective_scan"), _toplevel("selective_update")

    def params(f):
        sig = f.__doc__.splitlines()[0]
        return [a.split(":")[0].strip() for a in sig[sig.index("(") + 1:sig.rindex(")")].split(",")]

    assert params(ss.forward) == ["u", "A", "B", "C", "D", "delta", "delta_bias", "h_init",
                                  "length", "padding_side"]
    assert params(ss.backward) == ["u", "A", "B", "C", "D", "delta", "delta_bias", "h", "h_init",
                                   "dout", "dh_last", "length", "padding_side"]
    assert params(su.apply) == ["u", "A", "B", "C", "D", "delta", "delta_bias", "h"]


@pytest.mark.parametrize("mutate,msg", [
    (lambda a: a.update(u=a["u"][0]), "u must be a 3D tensor"),
    (lambda a: a.update(D=a["D"][None]), "D must be a 1D tensor"),
    (lambda a: a.update(A=torch.randn(4, 257)), "selective_scan only supports state_dim <= 256"),
    (lambda a: None, "u must be a CUDA tensor"),
])
def test_toplevel_scan_module_validation(mutate, msg):
    """The top-level module raises RuntimeError with the reference's messages
    (csrc/selective_scan/selective_scan.cpp:15-32,251) before any launch."""
    ss = _toplevel("selective_scan")
    a = _scan_args()
    mutate(a)
    with pytest.raises(RuntimeError, match=msg):
        ss.forward(a["u"], a["A"], a["B"], a["C"], a["D"], a["delta"], a["delta_bias"])
    h = torch.zeros(2, 4, 1, 6)
    with pytest.raises(RuntimeError, match=msg):
        ss.backward(a["u"], a["A"], a["B"], a["C"], a["D"], a["delta"], a["delta_bias"], h, None,
                    a["u"] if a["u"].dim() == 3 else torch.zeros(2, 4, 8), None)


def test_layer_chain_arguments_are_checked():
    """ssm_decode_layers validates its shapes and workspace before any launch;
    placeholder addresses stand in for the device buffers (no GPU needed)."""
    from ssm_mamba_amd import _native as N
    lib = N.lib()
    P = 4096  # never dereferenced: every call below fails its argument checks
    ws = lib.ssm_decode_layers_workspace(4, 48, 1024, 2048, 96, N.SSM_BF16)
    # the sync area (3 lines of 256 B), then per layer 8-byte units of 2 bf16
    # (x: 4 x 1024; xc, z, y: 4 x 2048) or 1 fp32 (partials: 128 blocks of
    # 4 x 96; their slice sums: 4 rows x 16 slices x 96, one slice per
    # state-update workgroup of 128 channels)
    per_layer = (4 * 1024 // 2 + 3 * 4 * 2048 // 2 + 128 * 4 * 96 + 4 * 16 * 96) * 8
    assert ws == 3 * 256 + 48 * per_layer
    assert lib.ssm_decode_layers_workspace(4, 48, 1024, 2047, 96, N.SSM_BF16) == 0
    assert lib.ssm_decode_layers_workspace(4, 0, 1024, 2048, 96, N.SSM_BF16) == 0
    args = lambda **kw: [kw.get(k, v) for k, v in dict(
        batch=4, nlayers=48, model_dim=1024, dim=2048, nstate=16, rank=64, width=4,
        dtype=N.SSM_BF16, table=P, x=P, out=P, eps=1e-5, ws=P * 64, ws_bytes=ws,
        stream=None).items()]
    call = lambda **kw: lib.ssm_decode_layers(*args(**kw))
    assert call(nstate=8) == 2 and b"nstate 16" in lib.ssm_last_error()
    assert call(rank=60) == 2 and b"rank" in lib.ssm_last_error()
    assert call(dim=2040) == 2 and b"folded x-projection" in lib.ssm_last_error()
    assert call(batch=9) == 2
    assert call(nlayers=0) == 1
    assert call(width=5) == 2 and b"width" in lib.ssm_last_error()
    assert call(ws_bytes=ws - 1) == 1 and b"workspace" in lib.ssm_last_error()
    assert call(model_dim=2048, ws_bytes=1 << 30) == 2 and b"single pass" in lib.ssm_last_error()
    assert call(dtype=N.SSM_F32, rank=64, ws_bytes=1 << 30) == 2 and b"at most 32" in lib.ssm_last_error()
    assert call(dtype=N.SSM_F32, rank=32, ws_bytes=1 << 30) == 2 and b"single pass" in lib.ssm_last_error()
    assert call(ws=P * 64 + 16) == 2 and b"256-byte" in lib.ssm_last_error()
    assert call(table=None) == 1


def test_layer_chain_keeps_every_table_it_built():
    """A HIP graph captured with one layer table keeps reading that table's
    address, so LayerChain.update() must not free it when the cache addresses
    change (another decoder's caches, a re-allocation): the old table stays
    alive and is reused when its addresses come back.  Host tensors stand in
    for the device ones (update() only builds the table of addresses)."""
    import gc
    import weakref

    from ssm_mamba_amd import decode as dec
    from ssm_mamba_amd.causal_lm import CausalLM, CausalLMConfig

    cfg = CausalLMConfig(vocab_size=64, model_dim=128, num_layers=2, device="cpu")
    m = CausalLM(cfg).to(torch.bfloat16).eval()
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    m.allocate_cache(2)
    chain = dec.LayerChain(m.layers, x)
    chain.update(m.layers)
    first = weakref.ref(chain.table)
    first_ptrs = chain.ptrs
    old = [(l.ssm._conv_context, l.ssm._ssm_hiddens) for l in m.layers]
    for l in m.layers:  # new caches, as a decoder of another max length would make
        l.ssm._conv_context = torch.zeros_like(l.ssm._conv_context)
        l.ssm._ssm_hiddens = torch.zeros_like(l.ssm._ssm_hiddens)
    chain.update(m.layers)
    assert chain.ptrs != first_ptrs
    gc.collect()
    assert first() is not None and first() is not chain.table
    assert len(chain.tables) == 2
    for l, (ctx, ssm) in zip(m.layers, old):
        l.ssm._conv_context, l.ssm._ssm_hiddens = ctx, ssm
    chain.update(m.layers)
    assert chain.table is first() and len(chain.tables) == 2
