"""ctypes binding of the C ABI in include/ssm_mamba.h (libssm_mamba_hip.so).

The library must have been built (``__graft_entry__.build()`` or
``python ssm-mamba_amd/_build.py``); there is no fallback implementation, so a
missing library raises immediately.
"""
from __future__ import annotations

import ctypes
import os
import threading

from ._build import LIB_PATH

_lock = threading.Lock()
_lib = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_sz = ctypes.c_size_t

SSM_F32 = 0
SSM_BF16 = 1
SSM_CHUNK = 16
SSM_REF_CHUNK = 128  # the reference's chunk (kernel_config.h:4-10): the pair layout's chunks
SSM_REF_SLOTS = SSM_REF_CHUNK // SSM_CHUNK
SSM_NOALLOC_SCRATCH_BYTES = 32 << 20

# exported symbol -> (restype, argtypes)
SIGNATURES = {
    "ssm_last_error": (ctypes.c_char_p, []),
    "ssm_abi_version": (_i32, []),
    "ssm_profile_begin": (_i32, []),
    "ssm_profile_end": (_i32, [ctypes.c_char_p, _sz]),
    "ssm_scan_nchunks": (_i64, [_i64]),
    "ssm_scan_ref_nchunks": (_i64, [_i64]),
    "ssm_scan_fwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "ssm_scan_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "ssm_selective_scan_fwd": (_i32, [
        _i64, _i64, _i64, _i64, _i32,          # batch, dim, seqlen, nstate, dtype
        _p, _p, _p, _p, _p, _i64,              # u, delta, A, B, C, bc_batch_stride
        _p, _p, _p, _p,                        # D, delta_bias, h_init, length
        _i32, _p, _i32,                        # padding_right, z, delta_softplus
        _p, _p, _p, _i32, _p,                  # out, out_ungated, h_chunks, h_pairs, h_last
        _p, _sz, _p,                           # workspace, bytes, stream
    ]),
    "ssm_selective_scan_fwd_noalloc": (_i32, [
        _i64, _i64, _i64, _i64, _i32,          # batch, dim, seqlen, nstate, dtype
        _p, _p, _p, _p, _p, _i64,              # u, delta, A, B, C, bc_batch_stride
        _p, _p, _p, _p,                        # D, delta_bias, h_init, length
        _i32, _p, _i32,                        # padding_right, z, delta_softplus
        _p, _p, _p, _i32, _p,                  # out, out_ungated, h_chunks, h_pairs, h_last
        _p,                                    # stream
    ]),
    "ssm_selective_scan_fwd_dt_proj": (_i32, [
        _i64, _i64, _i64, _i64, _i64, _i32,    # batch, dim, seqlen, nstate, dt_rank, dtype
        _p, _p, _i64, _p,                      # u, ssm_params, params_batch_stride, dt_weight
        _p, _p, _p, _p, _p,                    # A, D, delta_bias, h_init, length
        _i32, _p, _i64, _i32,                  # padding_right, z, z_batch_stride, delta_softplus
        _p, _p, _p,                            # out, delta_out, h_last
        _p, _sz, _p,                           # workspace, bytes, stream
    ]),
    "ssm_selective_scan_fwd_dt_proj_supported": (_i32, [_i64, _i64, _i64, _i64, _i64, _i32]),
    "ssm_selective_scan_bwd": (_i32, [
        _i64, _i64, _i64, _i64, _i32,
        _p, _p, _p, _p, _p, _i64,              # u, delta, A, B, C, bc_batch_stride
        _p, _p, _p, _p,                        # D, delta_bias, h_init, length
        _i32, _p, _p, _i32,                    # padding_right, z, out_ungated, delta_softplus
        _p, _i32, _p, _p,                      # h_chunks, h_pairs, dout, dh_last
        _p, _p, _p, _p, _p, _p, _p, _p, _p,    # du, ddelta, dA, dB, dC, dD, ddelta_bias, dh_init, dz
        _p, _sz, _p,                           # workspace, bytes, stream
    ]),
    "ssm_selective_state_update": (_i32, [
        _i64, _i64, _i64, _i32,                # batch, dim, nstate, dtype
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,  # state, new_state, x, dt, A, B, C, D, dt_bias, z
        _i32, _p, _p,                          # dt_softplus, out, stream
    ]),
    "ssm_causal_conv1d_fwd": (_i32, [
        _i64, _i64, _i64, _i64, _i32,          # batch, dim, seqlen, width, dtype
        _p, _i64, _p, _p, _i32, _p,            # x, x_batch_stride, weight, bias, silu, out
        _p, _p, _p,                            # lengths, window, stream
    ]),
    "ssm_causal_conv1d_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "ssm_causal_conv1d_bwd": (_i32, [
        _i64, _i64, _i64, _i64, _i32,
        _p, _p, _p, _p, _i32,                  # x, weight, bias, dout, silu
        _p, _p, _p,                            # dx, dweight, dbias
        _p, _sz, _p,                           # workspace, bytes, stream
    ]),
    "ssm_decode_gemv": (_i32, [
        _i64, _i64, _i64, _i32,                # batch, out_dim, in_dim, dtype
        _p, _p, _p, ctypes.c_float,            # weight, x, norm_weight, norm_eps
        _p, _p, _p, _p,                        # bias, residual, y, stream
    ]),
    "ssm_decode_in_proj_conv": (_i32, [
        _i64, _i64, _i64, _i64, _i32,          # batch, dim, in_dim, width, dtype
        _p, _p, _p, ctypes.c_float, _p,        # in_proj_weight, x, norm_weight, norm_eps, in_proj_bias
        _p, _p, _p,                            # conv_weight, conv_bias, window
        _p, _p,                                # xz, xc
        _p, _i64, _p,                          # x_proj_weight, params_dim, xproj_partials
        _p,                                    # stream
    ]),
    "ssm_decode_xproj_blocks": (_i64, [_i64, _i64]),
    "ssm_decode_ssm_step": (_i32, [
        _i64, _i64, _i64, _i64, _i32,          # batch, dim, nstate, rank, dtype
        _p, _i64,                              # params, params_blocks
        _p, _p, _p, _p,                        # dt_proj_weight, dt_bias, log_A, D
        _p, _p, _i64,                          # xc, xz, ld_xz
        _p, _p, _p,                            # state, y, stream
    ]),
    "ssm_decode_layers_workspace": (_i64, [_i64, _i64, _i64, _i64, _i64, _i32]),
    "ssm_decode_layers": (_i32, [
        _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32,  # batch, nlayers, model_dim, dim, nstate, rank, width, dtype
        _p, _p, _p, ctypes.c_float,            # layer_table, x, out, norm_eps
        _p, _i64, _p,                          # workspace, workspace_bytes, stream
    ]),
    "ssm_decode_layers_status": (_i32, [_p, _i64, _p]),
    "ssm_decode_pick_workspace": (_i64, [_i64]),
    "ssm_decode_pick": (_i32, [
        _i64, _i64, _i32, _p, _p,              # batch, vocab, dtype, probs, token
        _p, _i64, _i64, _p,                    # tokens, tokens_ld, tokens_cols, pos
        _p, _i64, _p,                          # workspace, workspace_bytes, stream
    ]),
    "ssm_rms_norm_cm": (_i32, [
        _i64, _i64, _i64, _i32,                # batch, channels, seqlen, dtype
        _p, _p, ctypes.c_float, _p, _p,        # x, weight, eps, out, stream
    ]),
}

ABI_VERSION = 10


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"ssm_mamba_amd: HIP library not found at {LIB_PATH}; build it with "
                    "`python -c 'import __graft_entry__ as g; g.build()'`")
            l = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                f = getattr(l, name)
                f.restype = res
                f.argtypes = args
            if l.ssm_abi_version() != ABI_VERSION:
                raise RuntimeError("ssm_mamba_amd: HIP library ABI version mismatch; rebuild it")
            _lib = l
    return _lib


def profile_begin() -> None:
    check(lib().ssm_profile_begin())


def profile_end() -> dict:
    """Returns {kernel: (launches, total_ms)} for the launches timed since
    profile_begin()."""
    buf = ctypes.create_string_buffer(8192)
    n = lib().ssm_profile_end(buf, len(buf))
    if n < 0:
        check(n)
    res = {}
    for line in buf.value.decode().splitlines():
        name, cnt, ms = line.split()
        res[name] = (int(cnt), float(ms))
    return res


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().ssm_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"ssm_mamba_amd: error code {rc}")
