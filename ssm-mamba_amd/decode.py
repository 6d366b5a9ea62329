"""Host side of the fused decode-step kernels (``ssm_decode_*`` in
include/ssm_mamba.h): one Mamba block step per token in three launches (four
when the x-projection cannot be folded) instead of the reference's per-op
sequence (``modules/block.py:80-86``, ``modules/mamba.py:189-243``), or the
steps of every layer of a model in one launch (``layers_step``), plus the
LM-head GEMV with the final RMSNorm (``models/causal_lm.py:93-104``).

These are inference kernels (no autograd).  ``block_step_supported`` says
whether a layer and an input qualify; callers fall back to the op-by-op path
otherwise.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native as N

_DTYPES = {torch.float32: N.SSM_F32, torch.bfloat16: N.SSM_BF16}
MAX_BATCH = 8
_STATE_SIZES = (4, 8, 16, 32, 64)

# The model harness takes the fused path whenever it qualifies; set False to
# force the op-by-op path (used to compare the two).
ENABLED = True
# Fold the x-projection into the in-projection and state-update kernels where
# ssm_decode_xproj_blocks allows; False keeps it a GEMV of its own.
FOLD_XPROJ = True
# CausalLM.step runs all of its layers in one launch (ssm_decode_layers) where
# layers_supported allows; False keeps three launches per layer.
LAYER_CHAIN = True


def _elems16(dtype: torch.dtype) -> int:
    return 16 // torch.empty((), dtype=dtype).element_size()


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _aligned(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0


def gemv(weight: torch.Tensor, x: torch.Tensor, norm_weight: Optional[torch.Tensor] = None,
         eps: float = 1e-6, bias: Optional[torch.Tensor] = None,
         residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = W @ v (+ bias) (+ residual) for x (batch, in) with v = x or, given
    norm_weight, the reference RMSNorm of x (scale 1 + norm_weight)."""
    batch, k = x.shape
    o = weight.shape[0]
    y = torch.empty(batch, o, device=x.device, dtype=x.dtype)
    with torch.cuda.device(x.device):
        N.check(N.lib().ssm_decode_gemv(batch, o, k, _DTYPES[x.dtype], weight.data_ptr(),
                                        x.data_ptr(), _ptr(norm_weight), float(eps), _ptr(bias),
                                        _ptr(residual), y.data_ptr(), _stream(x.device)))
    return y


def xproj_blocks(dim: int, params_dim: int) -> int:
    """Partial blocks of the folded x-projection (0: it does not apply)."""
    return int(N.lib().ssm_decode_xproj_blocks(dim, params_dim))


def in_proj_conv(weight: torch.Tensor, x: torch.Tensor, norm_weight: Optional[torch.Tensor],
                 eps: float, bias: Optional[torch.Tensor], conv_weight: torch.Tensor,
                 conv_bias: Optional[torch.Tensor], window: torch.Tensor,
                 x_proj_weight: Optional[torch.Tensor] = None):
    """(xz (batch, 2*dim), xc (batch, dim)) of the in-projection and conv step;
    the conv window advances in place.  With x_proj_weight (params_dim, dim)
    also the fp32 x-projection partials (P, batch, params_dim rounded up to 4)
    as a third output, for ssm_step."""
    batch, k = x.shape
    dim = weight.shape[0] // 2
    width = conv_weight.shape[-1]
    xz = torch.empty(batch, 2 * dim, device=x.device, dtype=x.dtype)
    xc = torch.empty(batch, dim, device=x.device, dtype=x.dtype)
    part, nout = None, 0
    if x_proj_weight is not None:
        nout = x_proj_weight.shape[0]
        nparts = xproj_blocks(dim, nout)
        if not nparts:
            raise RuntimeError(f"the x-projection cannot be folded at dim {dim}, params_dim {nout}")
        part = torch.empty(nparts, batch, (nout + 3) // 4 * 4, device=x.device, dtype=torch.float32)
    with torch.cuda.device(x.device):
        N.check(N.lib().ssm_decode_in_proj_conv(batch, dim, k, width, _DTYPES[x.dtype],
                                                weight.data_ptr(), x.data_ptr(), _ptr(norm_weight),
                                                float(eps), _ptr(bias), conv_weight.data_ptr(),
                                                _ptr(conv_bias), window.data_ptr(), xz.data_ptr(),
                                                xc.data_ptr(), _ptr(x_proj_weight), nout,
                                                _ptr(part), _stream(x.device)))
    return (xz, xc) if part is None else (xz, xc, part)


def ssm_step(params: torch.Tensor, rank: int, dt_proj_weight: torch.Tensor,
             dt_bias: Optional[torch.Tensor], log_A: torch.Tensor, D: Optional[torch.Tensor],
             xc: torch.Tensor, xz: torch.Tensor, state: torch.Tensor) -> torch.Tensor:
    """y (batch, dim) of the state update + gate; state advances in place.
    params is (batch, rank + 2*nstate), or the 3-d fp32 partials of
    in_proj_conv."""
    batch, dim = xc.shape
    nstate = state.shape[-1]
    blocks = params.shape[0] if params.dim() == 3 else 0
    y = torch.empty_like(xc)
    with torch.cuda.device(xc.device):
        N.check(N.lib().ssm_decode_ssm_step(batch, dim, nstate, rank, _DTYPES[xc.dtype],
                                            params.data_ptr(), blocks, dt_proj_weight.data_ptr(),
                                            _ptr(dt_bias), log_A.data_ptr(), _ptr(D),
                                            xc.data_ptr(), xz.data_ptr(), xz.stride(0),
                                            state.data_ptr(), y.data_ptr(), _stream(xc.device)))
    return y


def gemv_supported(weight: torch.Tensor, x: torch.Tensor, *others) -> bool:
    if not ENABLED or torch.is_grad_enabled():
        return False
    if not (x.is_cuda and x.dim() == 2 and x.dtype in _DTYPES and 1 <= x.shape[0] <= MAX_BATCH):
        return False
    e = _elems16(x.dtype)
    k = x.shape[1]
    if k % e or weight.dim() != 2 or weight.shape[1] != k:
        return False
    for t in (weight, x) + tuple(o for o in others if o is not None):
        if t.dtype != x.dtype or not t.is_contiguous() or t.device != x.device:
            return False
    return _aligned(weight) and _aligned(x) and all(_aligned(o) for o in others if o is not None)


def block_step_supported(ssm, x: torch.Tensor, norm_weight: Optional[torch.Tensor]) -> bool:
    """Whether the fused kernels can run Mamba ``ssm`` on the token batch x."""
    if torch.is_grad_enabled():
        return False
    ctx, state = ssm._conv_context, ssm._ssm_hiddens
    if ctx is None or state is None:
        return False
    inner = ssm.inner_dim
    batch = x.shape[0] if x.dim() == 2 else 0
    e = _elems16(x.dtype) if x.dtype in _DTYPES else 0
    if not e or not (2 <= ssm.conv_kernel <= 8) or ssm.state_dim not in _STATE_SIZES:
        return False
    if inner % e or ssm.delta_rank + 2 * ssm.state_dim > 16384:
        return False
    params = [ssm.input_proj.weight, ssm.input_proj.bias, ssm.conv.weight, ssm.conv.bias,
              ssm.ssm_param_proj.weight, ssm.delta_proj.weight, ssm.delta_proj.bias, ssm.log_A,
              ssm.D, ssm.out_proj.weight, ssm.out_proj.bias, norm_weight]
    if not gemv_supported(ssm.input_proj.weight, x, *params):
        return False
    if tuple(ctx.shape) != (batch, inner, ssm.conv_kernel - 1) or ctx.dtype != x.dtype \
            or not ctx.is_contiguous():
        return False
    if tuple(state.shape) != (batch, inner, ssm.state_dim) or state.dtype != torch.float32 \
            or not state.is_contiguous() or not _aligned(state):
        return False
    return True


def block_step(ssm, x: torch.Tensor, norm_weight: Optional[torch.Tensor] = None,
               eps: float = 1e-6, residual: bool = False) -> torch.Tensor:
    """Mamba.step(norm(x)) (+ x when residual): the fused path of
    ``Block.step`` (norm_weight and residual given) or ``Mamba.step``."""
    wx = ssm.ssm_param_proj.weight
    if FOLD_XPROJ and xproj_blocks(ssm.inner_dim, wx.shape[0]):
        xz, xc, params = in_proj_conv(ssm.input_proj.weight, x, norm_weight, eps,
                                      ssm.input_proj.bias, ssm.conv.weight, ssm.conv.bias,
                                      ssm._conv_context, x_proj_weight=wx)
    else:
        xz, xc = in_proj_conv(ssm.input_proj.weight, x, norm_weight, eps, ssm.input_proj.bias,
                              ssm.conv.weight, ssm.conv.bias, ssm._conv_context)
        params = gemv(wx, xc)                                             # (batch, R + 2N)
    y = ssm_step(params, ssm.delta_rank, ssm.delta_proj.weight, ssm.delta_proj.bias, ssm.log_A,
                 ssm.D, xc, xz, ssm._ssm_hiddens)
    return gemv(ssm.out_proj.weight, y, bias=ssm.out_proj.bias, residual=x if residual else None)


# ---- the layer chain: every layer's step in one launch ------------------------

_CHAIN_STATE = 16
_CHAIN_MAX_WIDTH = 4
_CHAIN_MAX_BATCH = 4


def _layer_tensors(block):
    """The SSM_LAYER_* row of one Block, in the header's order."""
    ssm = block.ssm
    return [ssm.input_proj.weight, ssm.input_proj.bias, block.norm.weight, ssm.conv.weight,
            ssm.conv.bias, ssm.ssm_param_proj.weight, ssm.delta_proj.weight, ssm.delta_proj.bias,
            ssm.log_A, ssm.D, ssm.out_proj.weight, ssm.out_proj.bias, ssm._conv_context,
            ssm._ssm_hiddens]


def layers_supported(layers, x: torch.Tensor) -> bool:
    """Whether ``layers_step`` can run the Blocks ``layers`` on the token batch
    x: every layer qualifies for the fused step, all share one shape and norm
    eps, the state size is 16 and the x-projection folds."""
    if not (ENABLED and LAYER_CHAIN and FOLD_XPROJ) or torch.is_grad_enabled() or len(layers) == 0:
        return False
    # up to 4 rows: the 8-row variants of the kernel spill registers
    if x.dim() != 2 or x.dtype not in _DTYPES or x.shape[0] > _CHAIN_MAX_BATCH:
        return False
    s0 = layers[0].ssm
    shape = (s0.inner_dim, s0.state_dim, s0.delta_rank, s0.conv_kernel)
    eps = layers[0].norm.eps
    if s0.state_dim != _CHAIN_STATE or not 2 <= s0.conv_kernel <= _CHAIN_MAX_WIDTH:
        return False
    e = _elems16(x.dtype)
    if s0.delta_rank % e or s0.delta_rank > 8 * e:
        return False
    # each projection in one pass: d_model up to 128 and d_inner up to 256
    # 16-byte chunks of elements
    if x.shape[1] > 128 * e or s0.inner_dim > 256 * e:
        return False
    if not xproj_blocks(s0.inner_dim, s0.delta_rank + 2 * s0.state_dim):
        return False
    for blk in layers:
        ssm = blk.ssm
        if (ssm.inner_dim, ssm.state_dim, ssm.delta_rank, ssm.conv_kernel) != shape \
                or blk.norm.eps != eps or blk.norm.weight is None:
            return False
        if not block_step_supported(ssm, x, blk.norm.weight):
            return False
        if ssm.conv.weight.shape[1] != 1:
            return False
    return True


class LayerChain:
    """The device-side layer table and the workspace of ``ssm_decode_layers``
    for one stack of Blocks and one (device, batch, dtype).  The table holds
    the layers' parameter and cache addresses.  When any of them changes the
    chain switches to the table for the new addresses, built once and kept
    in ``tables`` for the chain's lifetime: a HIP graph that captured a
    launch bakes in the address of the table it used, so no table is ever
    freed while the chain lives (a graph replayed after the addresses changed
    still reads the layer pointers it was captured with)."""

    def __init__(self, layers, x: torch.Tensor):
        s0 = layers[0].ssm
        self.batch, self.model_dim = x.shape
        self.dim, self.rank, self.width = s0.inner_dim, s0.delta_rank, s0.conv_kernel
        self.dtype, self.device = x.dtype, x.device
        self.eps = float(layers[0].norm.eps)
        nbytes = int(N.lib().ssm_decode_layers_workspace(
            self.batch, len(layers), self.model_dim, self.dim, self.rank + 2 * _CHAIN_STATE,
            _DTYPES[x.dtype]))
        if nbytes <= 0:
            raise RuntimeError("ssm_decode_layers_workspace rejected the shape")
        # zero-filled before the first launch (a launch counter and the
        # layers' hand-off buffers, whose flags must not match a launch yet)
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=x.device)
        self.ptrs = None
        self.table = None
        self.tables = {}  # pointer tuple -> device table; never pruned

    def update(self, layers) -> None:
        ptrs = tuple(0 if t is None else t.data_ptr() for blk in layers for t in _layer_tensors(blk))
        if ptrs != self.ptrs:
            table = self.tables.get(ptrs)
            if table is None:
                table = self.tables[ptrs] = torch.tensor(ptrs, dtype=torch.int64).to(self.device)
            self.table = table
            self.ptrs = ptrs

    def step(self, layers, x: torch.Tensor) -> torch.Tensor:
        self.update(layers)
        out = torch.empty_like(x)
        with torch.cuda.device(x.device):
            N.check(N.lib().ssm_decode_layers(
                self.batch, len(layers), self.model_dim, self.dim, _CHAIN_STATE, self.rank,
                self.width, _DTYPES[x.dtype], self.table.data_ptr(), x.data_ptr(), out.data_ptr(),
                self.eps, self.workspace.data_ptr(), self.workspace.numel(), _stream(x.device)))
        return out

    def check(self) -> None:
        """Synchronise and raise if a grid barrier of an earlier launch timed
        out (the outputs since the last check are then invalid)."""
        with torch.cuda.device(self.device):
            N.check(N.lib().ssm_decode_layers_status(self.workspace.data_ptr(),
                                                     self.workspace.numel(),
                                                     _stream(self.device)))


def layers_step(owner, layers, x: torch.Tensor) -> torch.Tensor:
    """x after Block.step of every layer in ``layers`` (one launch); the
    layers' caches advance in place.  ``owner`` keeps the LayerChain objects
    (one per device, batch and dtype)."""
    chains = owner.__dict__.setdefault("_layer_chains", {})
    key = (x.device, x.shape[0], x.dtype)
    chain = chains.get(key)
    if chain is None:
        chain = chains[key] = LayerChain(layers, x)
    return chain.step(layers, x)


_PICK_WS = {}


def pick_supported(probs: torch.Tensor) -> bool:
    return (ENABLED and probs.is_cuda and probs.dim() == 2 and probs.dtype in _DTYPES
            and 1 <= probs.shape[0] <= MAX_BATCH and probs.is_contiguous() and _aligned(probs)
            and probs.shape[1] * probs.element_size() % 16 == 0)


def pick(probs: torch.Tensor, token: torch.Tensor, tokens: Optional[torch.Tensor] = None,
         pos: Optional[torch.Tensor] = None) -> None:
    """token[:] = probs.argmax(-1) (first maximum, NaN highest, as torch), and
    with tokens and pos: tokens[:, min(pos, cols - 1)] = token; pos += 1 --
    one launch (int64 token (batch,), tokens (batch, cols), pos (1,))."""
    batch, vocab = probs.shape
    for t in (token, tokens, pos):
        if t is not None and (t.dtype != torch.int64 or t.device != probs.device):
            raise ValueError("pick: token, tokens and pos must be int64 on the probs' device")
    if token.numel() != batch or not token.is_contiguous():
        raise ValueError("pick: token must be a contiguous (batch,) tensor")
    if tokens is not None and (tokens.shape[0] != batch or tokens.stride(1) != 1):
        raise ValueError("pick: tokens must be (batch, cols) with unit column stride")
    # the counter the last workgroup leaves at zero, kept per device (the
    # graph a GreedyDecoder captures bakes its address in)
    ws = _PICK_WS.get(probs.device)
    need = int(N.lib().ssm_decode_pick_workspace(MAX_BATCH))
    if ws is None:
        ws = _PICK_WS[probs.device] = torch.zeros(need, dtype=torch.uint8, device=probs.device)
    with torch.cuda.device(probs.device):
        N.check(N.lib().ssm_decode_pick(
            batch, vocab, _DTYPES[probs.dtype], probs.data_ptr(), token.data_ptr(), _ptr(tokens),
            tokens.stride(0) if tokens is not None else 0,
            tokens.shape[1] if tokens is not None else 0, _ptr(pos), ws.data_ptr(), ws.numel(),
            _stream(probs.device)))


def layers_check(owner) -> None:
    """Raise if any layer-chain launch of ``owner`` hit a barrier time-out."""
    for chain in owner.__dict__.get("_layer_chains", {}).values():
        chain.check()
