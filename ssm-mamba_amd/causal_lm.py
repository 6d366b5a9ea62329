"""Mamba causal language model over the MI355X selective-scan operators.

Module tree, parameter names, shapes, initialisation and the public methods
follow the reference, so a reference ``state_dict`` loads unchanged and
callers see the same API:

* ``RMSNorm``        -- ``modules/rms_norm.py:4-31`` (scale ``1 + weight``);
* ``Mamba``          -- ``modules/mamba.py:9-243`` (``forward`` :82-187,
  ``step`` :189-243);
* ``Block``          -- ``modules/block.py:8-87``;
* ``CausalLMConfig`` / ``CausalLM`` -- ``models/causal_lm.py:9-134``.

Layout.  Inside the layer stack activations stay channel-major,
(batch, channels, seq_len), which is the layout the scan kernels stream.
Every projection is computed as ``W @ X`` on channel-major ``X`` (one batched
GEMM with the weight broadcast over the batch), so the reference's per-layer
permute copies (``modules/mamba.py:104-111,156-163,181``) do not exist here:
the sequence is transposed once after the embedding and once before the LM
head.  The z gate is fused into the scan / state-update kernels.  In an
inference prefill (bf16 on the GPU) the in-projection is one GEMM whose x and
z halves the conv and scan kernels read in place, the x-projection output is
token-major, the reference's own layout of ssm_params, and the step-size
projection runs inside the scan kernels (``ssm_selective_scan_fwd_dt_proj``),
which read dt, B and C from it in place.

Decode.  ``Mamba.step`` updates the per-layer caches in place (conv window and
fp32 SSM state), so a whole token step -- all layers, final norm, LM head and
the greedy pick -- can be captured once in a HIP graph and replayed per token
(``GreedyDecoder``).  ``CausalLM.generate`` returns exactly the reference's
sequences (``models/causal_lm.py:98-133``), including its EOS handling.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Literal, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native as _N
from . import decode as _dec
from .causal_conv1d import causal_conv1d_fn
from .ops import selective_scan_fn, selective_state_update

_DTYPES = {torch.float32: _N.SSM_F32, torch.bfloat16: _N.SSM_BF16}

__all__ = ["RMSNorm", "Mamba", "Block", "CausalLMConfig", "CausalLM", "GreedyDecoder"]


def _proj_cm(weight: torch.Tensor, x: torch.Tensor, bias: Optional[torch.Tensor] = None):
    """``weight @ x`` for channel-major x (batch, in, L) -> (batch, out, L):
    one strided-batched GEMM with the weight broadcast over the batch (batch
    stride 0), contiguous result.  (``torch.matmul`` would fold a weight that
    requires grad through transposed copies of x and of the result.)  A view
    whose per-batch (in, L) matrices are contiguous, such as a channel slice
    of a larger activation, is passed as it is: the GEMM takes its batch
    stride."""
    if not (x.stride(2) == 1 and x.stride(1) == x.shape[2]):
        x = x.contiguous()
    w = weight.expand(x.shape[0], weight.shape[0], weight.shape[1])
    if bias is None:
        return torch.bmm(w, x)
    return torch.baddbmm(bias[None, :, None].expand(x.shape[0], weight.shape[0], x.shape[2]), w, x)


def rms_norm_cm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the channel axis of channel-major x (batch, channels, L) in
    one HIP kernel (inference: no autograd)."""
    x = x.contiguous()
    out = torch.empty_like(x)
    batch, ch, seqlen = x.shape
    with torch.cuda.device(x.device):
        _N.check(_N.lib().ssm_rms_norm_cm(batch, ch, seqlen, _DTYPES[x.dtype], x.data_ptr(),
                                          weight.contiguous().data_ptr(), float(eps),
                                          out.data_ptr(),
                                          torch.cuda.current_stream(x.device).cuda_stream))
    return out


def causal_conv_silu(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                     window: Optional[torch.Tensor] = None,
                     lengths: Optional[torch.Tensor] = None):
    """silu(causal depthwise conv1d(x)) over channel-major x (batch, channels, L)
    in one HIP kernel: ``modules/mamba.py:138-139`` (left zero padding of k-1,
    keep the first L); ``window`` receives the decode conv cache."""
    return causal_conv1d_fn(x, weight, bias, activation="silu", window=window, lengths=lengths)


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) * (1 + weight), computed in float32 and cast
    back to x's dtype (``modules/rms_norm.py:4-31``).  ``dim`` selects the
    normalised axis (-1 for token-major input, 1 for channel-major)."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.zeros(dim))

    def forward(self, x: torch.Tensor, dim: int = -1) -> torch.Tensor:
        if (dim % x.dim() == 1 and x.dim() == 3 and x.is_cuda and not torch.is_grad_enabled()
                and x.dtype in (torch.float32, torch.bfloat16) and self.weight.dtype == x.dtype):
            return rms_norm_cm(x, self.weight, self.eps)
        xf = x.float()
        d = dim % x.dim()
        scale = torch.rsqrt(xf.pow(2).mean(d, keepdim=True) + self.eps)
        w = 1.0 + self.weight.float()
        if d != x.dim() - 1:
            w = w.view(-1, *([1] * (x.dim() - 1 - d)))
        return (xf * scale * w).type_as(x)


class Mamba(nn.Module):
    """Selective-SSM mixer (``modules/mamba.py:9-243``)."""

    def __init__(
        self,
        model_dim: int = 512,
        state_dim: int = 16,
        conv_kernel: int = 4,
        expansion_factor: int = 2,
        delta_rank: int | str = "auto",
        delta_min: float = 0.001,
        delta_max: float = 0.1,
        delta_init: Literal["random", "constant"] = "random",
        delta_scale: float = 1.0,
        delta_init_floor: float = 1e-4,
        conv_bias: bool = False,
        bias: bool = False,
        device: str | None = None,
    ):
        super().__init__()
        self.model_dim = model_dim
        self.state_dim = state_dim
        self.inner_dim = expansion_factor * model_dim
        self.conv_kernel = conv_kernel
        self.delta_rank = math.ceil(model_dim / 16) if delta_rank == "auto" else delta_rank
        self.conv_bias = conv_bias
        inner, rank, nstate = self.inner_dim, self.delta_rank, state_dim

        self.input_proj = nn.Linear(model_dim, 2 * inner, bias=bias, device=device)
        self.conv = nn.Conv1d(inner, inner, kernel_size=conv_kernel, padding=conv_kernel - 1,
                              groups=inner, bias=conv_bias, device=device)
        self.ssm_param_proj = nn.Linear(inner, rank + 2 * nstate, bias=False, device=device)
        self.delta_proj = nn.Linear(rank, inner, bias=True, device=device)

        # Initialisation of the step-size projection (modules/mamba.py:52-69):
        # weight constant or uniform at rank^-0.5 * scale; bias = softplus^-1
        # of a log-uniform step in [delta_min, delta_max], floored.
        std = rank ** -0.5 * delta_scale
        with torch.no_grad():
            if delta_init == "constant":
                self.delta_proj.weight.fill_(std)
            elif delta_init == "random":
                self.delta_proj.weight.uniform_(-std, std)
            else:
                raise NotImplementedError
            lo, hi = math.log(delta_min), math.log(delta_max)
            dt = torch.exp(torch.rand(inner, device=device) * (hi - lo) + lo)
            dt = dt.clamp(min=delta_init_floor)
            self.delta_proj.bias.copy_(dt + torch.log(-torch.expm1(-dt)))

        # S4D-real A = -(1..N) per channel, stored as its log (modules/mamba.py:71-73)
        steps = torch.arange(1, nstate + 1, dtype=torch.float32, device=device)
        self.log_A = nn.Parameter(torch.log(steps).repeat(inner, 1))
        self.D = nn.Parameter(torch.ones(inner, device=device))
        self.out_proj = nn.Linear(inner, model_dim, bias=bias, device=device)

        self._ssm_hiddens: Optional[torch.Tensor] = None   # (batch, inner, N) float32
        self._conv_context: Optional[torch.Tensor] = None  # (batch, inner, k-1)
        self._param_cache = None
        self._xproj_t = None

    def _scan_params(self):
        """(A, D, delta_bias) for the scan: A = -exp(log_A) (``modules/mamba.py:166``)
        and D / delta_bias in float32.  Without autograd they are kept and
        recomputed only when a parameter changes (its version counter, storage,
        dtype or device), so an inference prefill runs no conversion kernels."""
        bias = self.delta_proj.bias
        if torch.is_grad_enabled():
            return -torch.exp(self.log_A.float()), self.D, bias
        key = tuple(None if t is None else (t._version, t.data_ptr(), t.dtype, t.device)
                    for t in (self.log_A, self.D, bias))
        if self._param_cache is None or self._param_cache[0] != key:
            self._param_cache = (key, -torch.exp(self.log_A.detach().float()),
                                 self.D.detach().float(),
                                 None if bias is None else bias.detach().float())
        return self._param_cache[1:]

    def _x_proj_t(self) -> torch.Tensor:
        """W_x^T (inner, R + 2N), contiguous, for the token-major x-projection
        xc^T W_x^T (the reference's layout of ssm_params, modules/mamba.py:
        141-145).  Kept until the weight changes, as in _scan_params."""
        w = self.ssm_param_proj.weight
        key = (w._version, w.data_ptr(), w.dtype, w.device)
        if self._xproj_t is None or self._xproj_t[0] != key:
            self._xproj_t = (key, w.detach().t().contiguous())
        return self._xproj_t[1]

    def _dt_fusable(self, x: torch.Tensor, h0: Optional[torch.Tensor],
                    lengths: Optional[torch.Tensor]) -> bool:
        """Whether a forward of x (batch, model_dim, L) takes the inference
        prefill path: the in-projection as one GEMM whose x and z halves are
        read in place, and the scan with the step-size projection fused in
        (ssm_selective_scan_fwd_dt_proj): no autograd, bf16 on the GPU, and a
        shape the fused kernel takes."""
        w_dt = self.delta_proj.weight
        if torch.is_grad_enabled() or not x.is_cuda or x.dtype != torch.bfloat16:
            return False
        if any(w.dtype != torch.bfloat16 for w in (w_dt, self.ssm_param_proj.weight,
                                                     self.input_proj.weight)):
            return False
        if not (w_dt.is_contiguous() and w_dt.data_ptr() % 16 == 0):
            return False
        batch, seqlen = x.shape[0], x.shape[2]
        if h0 is not None and tuple(h0.shape) != (batch, self.inner_dim, self.state_dim):
            return False
        if lengths is not None and lengths.device != x.device:
            return False
        return bool(_N.lib().ssm_selective_scan_fwd_dt_proj_supported(
            batch, self.inner_dim, seqlen, self.state_dim, self.delta_rank, _N.SSM_BF16))

    def _scan_dt_proj(self, xc: torch.Tensor, z: torch.Tensor, h0: Optional[torch.Tensor],
                      lengths: Optional[torch.Tensor]):
        """modules/mamba.py:141-171 for inference: the token-major x-projection
        (one GEMM), then the scan with delta_raw = W_dt dt computed by the scan
        kernels' producers on the matrix cores and B, C read in place from the
        projection output (no delta or channel-major B/C tensors).  z may be
        the gate half of the in-projection output (its batch stride is taken).
        Returns (out, last state)."""
        batch, inner, seqlen = xc.shape
        nstate, rank = self.state_dim, self.delta_rank
        w_xt = self._x_proj_t()
        params = torch.bmm(xc.transpose(1, 2), w_xt.expand(batch, *w_xt.shape))  # (batch, L, P)
        A, D, dt_bias = self._scan_params()
        h0 = None if h0 is None else h0.detach().float().contiguous()
        lengths = None if lengths is None else lengths.to(torch.int64).contiguous()
        out = torch.empty_like(xc)
        last = torch.empty(batch, inner, nstate, dtype=torch.float32, device=xc.device)
        assert z.stride(2) == 1 and z.stride(1) == seqlen
        zbs = 0 if batch == 1 else z.stride(0)
        lib = _N.lib()
        ws = torch.empty(lib.ssm_scan_fwd_workspace_bytes(batch, inner, seqlen, nstate),
                         dtype=torch.uint8, device=xc.device)
        ptr = lambda t: None if t is None else t.data_ptr()
        with torch.cuda.device(xc.device):
            _N.check(lib.ssm_selective_scan_fwd_dt_proj(
                batch, inner, seqlen, nstate, rank, _N.SSM_BF16, xc.data_ptr(), params.data_ptr(),
                0, self.delta_proj.weight.data_ptr(), A.data_ptr(), ptr(D), ptr(dt_bias), ptr(h0),
                ptr(lengths), 0, z.data_ptr(), zbs, 1, out.data_ptr(), None, last.data_ptr(),
                ws.data_ptr(), ws.numel(), torch.cuda.current_stream(xc.device).cuda_stream))
        return out, last

    # ---- caches ---------------------------------------------------------
    def allocate_cache(self, batch: int, device=None, dtype=None) -> None:
        """Pre-allocate the decode caches.  Later prefills with use_cache=True
        write into these buffers in place, so their addresses stay fixed (a
        captured decode graph stays valid across prompts of this batch size)."""
        w = self.input_proj.weight
        device = w.device if device is None else device
        dtype = w.dtype if dtype is None else dtype
        ctx_shape = (batch, self.inner_dim, self.conv_kernel - 1)
        ssm_shape = (batch, self.inner_dim, self.state_dim)
        ctx, ssm = self._conv_context, self._ssm_hiddens
        if not (ctx is not None and tuple(ctx.shape) == ctx_shape and ctx.dtype == dtype
                and ctx.device == torch.device(device)):
            self._conv_context = torch.zeros(ctx_shape, device=device, dtype=dtype)
        if not (ssm is not None and tuple(ssm.shape) == ssm_shape and ssm.is_contiguous()
                and ssm.dtype == torch.float32
                and ssm.device == torch.device(device)):
            self._ssm_hiddens = torch.zeros(ssm_shape, device=device, dtype=torch.float32)

    @staticmethod
    def _keep(old: Optional[torch.Tensor], new: torch.Tensor) -> torch.Tensor:
        if (old is not None and old.shape == new.shape and old.dtype == new.dtype
                and old.device == new.device):
            old.copy_(new)
            return old
        return new.clone(memory_format=torch.contiguous_format)

    def _conv_window(self, xs: torch.Tensor) -> torch.Tensor:
        """The buffer a prefill's conv kernel fills with the decode conv cache:
        the existing cache when it fits (its address stays fixed for a captured
        decode graph), else a new one."""
        shape = (xs.shape[0], xs.shape[1], self.conv_kernel - 1)
        ctx = self._conv_context
        if (ctx is not None and tuple(ctx.shape) == shape and ctx.dtype == xs.dtype
                and ctx.device == xs.device and ctx.is_contiguous()):
            return ctx
        return torch.empty(shape, device=xs.device, dtype=xs.dtype)

    # ---- prefill / training ----------------------------------------------
    def forward(self, hidden_states: torch.Tensor, ssm_hiddens: Optional[torch.Tensor] = None,
                lengths: Optional[torch.Tensor] = None, use_cache: bool = False):
        """hidden_states (batch, seq_len, model_dim) -> ((batch, seq_len,
        model_dim), last_ssm_hiddens (batch, inner, N)), as
        ``modules/mamba.py:82-187``."""
        y, last = self.forward_cm(hidden_states.transpose(1, 2).contiguous(), ssm_hiddens,
                                  lengths, use_cache)
        return y.transpose(1, 2).contiguous(), last

    def forward_cm(self, x: torch.Tensor, ssm_hiddens: Optional[torch.Tensor] = None,
                   lengths: Optional[torch.Tensor] = None, use_cache: bool = False,
                   residual: Optional[torch.Tensor] = None, residual_inplace: bool = False):
        """Channel-major forward: x (batch, model_dim, L) -> (batch, model_dim, L)
        (plus ``residual`` when given, added by the out-projection GEMM) and
        the last SSM state."""
        inner, rank, nstate = self.inner_dim, self.delta_rank, self.state_dim
        w_in, b_in = self.input_proj.weight, self.input_proj.bias
        fused = self._dt_fusable(x, ssm_hiddens, lengths)
        if fused:
            # one GEMM for both halves; the conv and the scan read them in place
            xz = _proj_cm(w_in, x, b_in)                                  # (batch, 2 inner, L)
            xs, z = xz[:, :inner], xz[:, inner:]
        else:
            xs = _proj_cm(w_in[:inner], x, None if b_in is None else b_in[:inner])
            z = _proj_cm(w_in[inner:], x, None if b_in is None else b_in[inner:])
        # with use_cache the conv kernel also leaves the k-1 pre-conv inputs
        # ending at position lengths-1 (zero before the row start), the
        # reference's conv cache (modules/mamba.py:113-135)
        window = self._conv_window(xs) if use_cache else None
        xc = causal_conv_silu(xs, self.conv.weight, self.conv.bias, window=window,
                              lengths=lengths if use_cache else None)
        if use_cache:
            self._conv_context = window
        # padding_side "left" is the reference's default at this call
        # (modules/mamba.py:170-175 passes no padding argument)
        if fused:
            y, last = self._scan_dt_proj(xc, z, ssm_hiddens, lengths)
        else:
            params = _proj_cm(self.ssm_param_proj.weight, xc)           # (batch, R + 2N, L)
            delta = _proj_cm(self.delta_proj.weight, params[:, :rank])
            # B and C go to the scan as slices of params (one shared batch stride)
            Bm = params[:, rank:rank + nstate]
            Cm = params[:, rank + nstate:]
            A, D, dt_bias = self._scan_params()
            y, last = selective_scan_fn(xc, delta, A, Bm, Cm, D, z=z, delta_bias=dt_bias,
                                        return_last_state=True, h_init=ssm_hiddens,
                                        length=lengths, padding_side="left")
        if use_cache:
            self._ssm_hiddens = self._keep(self._ssm_hiddens, last.detach())
        if residual is not None and self.out_proj.bias is None:
            w = self.out_proj.weight.expand(y.shape[0], *self.out_proj.weight.shape)
            if residual_inplace:
                out = residual.baddbmm_(w, y)       # the stream is updated in place
            else:
                out = torch.baddbmm(residual, w, y)
        else:
            out = _proj_cm(self.out_proj.weight, y, self.out_proj.bias)
            if residual is not None:
                out = residual + out
        return out, last

    # ---- decode ----------------------------------------------------------
    def step(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """One token (batch, model_dim) -> (batch, model_dim); updates the conv
        window and the SSM state in place (``modules/mamba.py:189-243``)."""
        if self._conv_context is None or self._ssm_hiddens is None:
            raise RuntimeError("Mamba.step needs the caches of a forward(use_cache=True) "
                               "or allocate_cache()")
        if _dec.block_step_supported(self, hidden_states, None):
            return _dec.block_step(self, hidden_states)
        inner, rank, nstate = self.inner_dim, self.delta_rank, self.state_dim
        w_in, b_in = self.input_proj.weight, self.input_proj.bias
        xs = F.linear(hidden_states, w_in[:inner], None if b_in is None else b_in[:inner])
        z = F.linear(hidden_states, w_in[inner:], None if b_in is None else b_in[inner:])
        ctx = self._conv_context
        window = torch.cat([ctx, xs[..., None]], dim=-1)              # (batch, inner, k)
        xc = (window * self.conv.weight[:, 0, :]).sum(dim=-1)
        if self.conv.bias is not None:
            xc = xc + self.conv.bias
        xc = F.silu(xc)
        ctx.copy_(window[..., 1:])
        params = F.linear(xc, self.ssm_param_proj.weight)             # (batch, R + 2N)
        delta = F.linear(params[:, :rank], self.delta_proj.weight)
        A = -torch.exp(self.log_A.float())
        out = selective_state_update(self._ssm_hiddens, xc, delta, A,
                                     params[:, rank:rank + nstate], params[:, rank + nstate:],
                                     self.D, z=z, dt_bias=self.delta_proj.bias)
        return F.linear(out, self.out_proj.weight, self.out_proj.bias)


class Block(nn.Module):
    """Pre-norm residual block: x + dropout(mamba(norm(x))) (``modules/block.py:8-87``)."""

    def __init__(
        self,
        model_dim: int = 512,
        state_dim: int = 16,
        expansion_factor: int = 2,
        conv_kernel: int = 4,
        conv_bias: bool = False,
        bias: bool = False,
        delta_rank: int | str = "auto",
        delta_min: float = 0.001,
        delta_max: float = 0.1,
        delta_init: str = "random",
        delta_scale: float = 1.0,
        delta_init_floor: float = 1e-4,
        dropout_rate: float = 0.15,
        device: str | None = None,
    ):
        super().__init__()
        self.norm = RMSNorm(model_dim)
        self.ssm = Mamba(model_dim=model_dim, state_dim=state_dim,
                         expansion_factor=expansion_factor, bias=bias, conv_kernel=conv_kernel,
                         conv_bias=conv_bias, delta_rank=delta_rank, delta_min=delta_min,
                         delta_max=delta_max, delta_init=delta_init, delta_scale=delta_scale,
                         delta_init_floor=delta_init_floor, device=device)
        self.dropout = nn.Dropout(dropout_rate)

    def forward(self, hidden_states: torch.Tensor, lengths: Optional[torch.Tensor] = None,
                ssm_hiddens: Optional[torch.Tensor] = None, use_cache: bool = False):
        """(batch, seq_len, model_dim) -> ((batch, seq_len, model_dim), last state)."""
        y, last = self.forward_cm(hidden_states.transpose(1, 2).contiguous(), lengths,
                                  ssm_hiddens, use_cache)
        return y.transpose(1, 2).contiguous(), last

    def forward_cm(self, x: torch.Tensor, lengths: Optional[torch.Tensor] = None,
                   ssm_hiddens: Optional[torch.Tensor] = None, use_cache: bool = False,
                   inplace: bool = False):
        """Channel-major block; with ``inplace`` (and no active dropout) the
        residual stream x itself receives x + mixer(norm(x))."""
        h = self.norm(x, dim=1)
        if not self.training or self.dropout.p == 0.0:
            # x + mixer(h) with the add in the out-projection GEMM (beta = 1)
            return self.ssm.forward_cm(h, ssm_hiddens=ssm_hiddens, lengths=lengths,
                                       use_cache=use_cache, residual=x,
                                       residual_inplace=inplace and not torch.is_grad_enabled())
        y, last = self.ssm.forward_cm(h, ssm_hiddens=ssm_hiddens, lengths=lengths,
                                      use_cache=use_cache)
        return x + self.dropout(y), last

    def step(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if _dec.block_step_supported(self.ssm, hidden_states, self.norm.weight):
            # norm, mixer and residual in the four fused decode kernels
            return _dec.block_step(self.ssm, hidden_states, self.norm.weight, self.norm.eps,
                                   residual=True)
        return hidden_states + self.ssm.step(self.norm(hidden_states))


@dataclass
class CausalLMConfig:
    """Same fields and defaults as ``models/causal_lm.py:9-30``."""
    vocab_size: int = 32000
    model_dim: int = 512
    state_dim: int = 16
    expansion_factor: int = 2
    conv_kernel: int = 4
    conv_bias: bool = False
    bias: bool = False
    delta_rank: int | str = "auto"
    delta_min: float = 0.001
    delta_max: float = 0.1
    delta_init: Literal["random", "constant"] = "random"
    delta_scale: float = 1.0
    delta_init_floor: float = 1e-4
    dropout_rate: float = 0.15
    num_layers: int = 5
    tie_embeddings: bool = True
    device: str | None = None
    pad_token_id: int = 0
    bos_token_id: int = 1
    eos_token_id: int = 2


def _greedy_pick(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """argmax of softmax(logits / temperature), as ``models/causal_lm.py:117-120``."""
    if temperature != 1.0:
        logits = logits / temperature
    return torch.softmax(logits, dim=-1).argmax(dim=-1)


class CausalLM(nn.Module):
    """Embedding -> Blocks -> RMSNorm -> LM head (``models/causal_lm.py:32-134``)."""

    def __init__(self, config: CausalLMConfig | None = None):
        super().__init__()
        if config is None:
            config = CausalLMConfig()
        self.config = config
        c = config
        self.embedding = nn.Embedding(c.vocab_size, c.model_dim, device=c.device)
        self.layers = nn.ModuleList([
            Block(model_dim=c.model_dim, state_dim=c.state_dim,
                  expansion_factor=c.expansion_factor, conv_kernel=c.conv_kernel,
                  conv_bias=c.conv_bias, bias=c.bias, delta_rank=c.delta_rank,
                  delta_min=c.delta_min, delta_max=c.delta_max, delta_init=c.delta_init,
                  delta_scale=c.delta_scale, delta_init_floor=c.delta_init_floor,
                  dropout_rate=c.dropout_rate, device=c.device)
            for _ in range(c.num_layers)
        ])
        self.norm = RMSNorm(c.model_dim)
        self.lm_head = nn.Linear(c.model_dim, c.vocab_size, bias=False, device=c.device)
        if c.tie_embeddings:
            self.lm_head.weight = self.embedding.weight
        self._decoders = {}

    def allocate_cache(self, batch: int) -> None:
        for layer in self.layers:
            layer.ssm.allocate_cache(batch)

    def forward(self, input_ids: torch.Tensor, lengths: Optional[torch.Tensor] = None,
                use_cache: bool = False) -> torch.Tensor:
        """input_ids (batch, seq_len) -> logits (batch, seq_len, vocab)."""
        x = self.embedding(input_ids).transpose(1, 2).contiguous()
        for layer in self.layers:
            # x is this method's own stream: layers may update it in place
            x, _ = layer.forward_cm(x, lengths=lengths, use_cache=use_cache, inplace=True)
        x = self.norm(x, dim=1).transpose(1, 2).contiguous()
        return self.lm_head(x)

    def forward_last(self, input_ids: torch.Tensor, lengths: Optional[torch.Tensor] = None,
                     use_cache: bool = False) -> torch.Tensor:
        """Logits at position lengths - 1 of each row, (batch, vocab): the rows
        of ``forward``'s logits that the reference's ``generate`` keeps
        (``models/causal_lm.py:104-113``, the same index, negative wrapping
        included).  The final norm and the LM head run on those rows only."""
        batch, seqlen = input_ids.shape
        x = self.embedding(input_ids).transpose(1, 2).contiguous()
        for layer in self.layers:
            x, _ = layer.forward_cm(x, lengths=lengths, use_cache=use_cache, inplace=True)
        last = (torch.full((batch,), seqlen, dtype=torch.long, device=input_ids.device)
                if lengths is None else lengths) - 1
        x = x[torch.arange(batch, device=x.device), :, last]  # (batch, model_dim)
        return self._head(x)

    def _head(self, x: torch.Tensor) -> torch.Tensor:
        """Final norm and LM head of (batch, model_dim) rows."""
        if _dec.gemv_supported(self.lm_head.weight, x, self.norm.weight):
            return _dec.gemv(self.lm_head.weight, x, norm_weight=self.norm.weight,
                             eps=self.norm.eps)
        return self.lm_head(self.norm(x))

    def step(self, input_ids: torch.Tensor) -> torch.Tensor:
        """input_ids (batch,) -> logits (batch, vocab), advancing every cache."""
        x = self.embedding(input_ids)
        if _dec.layers_supported(self.layers, x):
            # every layer's step in one launch
            x = _dec.layers_step(self, self.layers, x)
            if not torch.cuda.is_current_stream_capturing():
                _dec.layers_check(self)
        else:
            for layer in self.layers:
                x = layer.step(x)
        return self._head(x)

    def decoder(self, batch: int, max_new_tokens: int, temperature: float = 1.0) -> "GreedyDecoder":
        key = (batch, max_new_tokens, float(temperature))
        dec = self._decoders.get(key)
        if dec is None:
            dec = GreedyDecoder(self, batch, max_new_tokens, temperature)
            self._decoders[key] = dec
        return dec

    def generate(self, input_ids: torch.Tensor, max_new_tokens: int = 100,
                 temperature: float = 1.0, use_graph: Optional[bool] = None) -> torch.Tensor:
        """Greedy generation with the reference's semantics
        (``models/causal_lm.py:98-133``): prompt lengths count the non-pad
        tokens, the first new token comes from the logits at lengths-1,
        generation stops once every row has produced EOS, and every position
        from a row's first EOS on is set to EOS.  With ``use_graph`` (default on
        a GPU) each token step is one HIP-graph replay."""
        if use_graph is None:
            use_graph = input_ids.is_cuda
        with torch.no_grad():
            if use_graph and max_new_tokens > 0:
                new = self.decoder(input_ids.shape[0], max_new_tokens, temperature).generate(input_ids)
            else:
                new = self._generate_eager(input_ids, max_new_tokens, temperature)
            eos = self.config.eos_token_id
            seq = torch.cat([input_ids, new], dim=1)
            after_eos = (seq == eos).to(torch.int32).cumsum(dim=1) >= 1
            return torch.where(after_eos, torch.full_like(seq, eos), seq)

    def _generate_eager(self, input_ids, max_new_tokens, temperature):
        batch = input_ids.shape[0]
        dev = input_ids.device
        lengths = (input_ids != self.config.pad_token_id).sum(dim=1)
        logits = self.forward_last(input_ids, lengths, use_cache=True)
        finished = torch.zeros(batch, dtype=torch.bool, device=dev)
        out = []
        for _ in range(max_new_tokens):
            nxt = _greedy_pick(logits, temperature)
            out.append(nxt)
            finished |= nxt == self.config.eos_token_id
            if bool(finished.all()):
                break
            logits = self.step(nxt)
        if not out:
            return input_ids.new_zeros(batch, 0)
        return torch.stack(out, dim=1)


class GreedyDecoder:
    """Greedy decoding with one token step -- every layer's ``step``, the final
    norm, the LM head and the pick -- captured in a HIP graph.

    The decoder owns static buffers: the per-layer caches (allocated once, and
    refilled in place by each prefill), the current token, the generated
    tokens and a device-side position counter, so a replay needs no host
    work.  Overlapping use of one model by two decoders of the same batch size
    shares the caches; run them one after the other."""

    def __init__(self, model: CausalLM, batch: int, max_new_tokens: int, temperature: float = 1.0):
        self.model = model
        self.batch = batch
        self.max_new = max_new_tokens
        self.temperature = temperature
        dev = model.embedding.weight.device
        self.device = dev
        model.allocate_cache(batch)
        # the graph bakes in these buffers' addresses: hold them, and put them
        # back on the layers before every prefill
        self.caches = [(layer.ssm._conv_context, layer.ssm._ssm_hiddens) for layer in model.layers]
        self.token = torch.zeros(batch, dtype=torch.long, device=dev)
        self.tokens = torch.zeros(batch, max(max_new_tokens, 1), dtype=torch.long, device=dev)
        self.pos = torch.zeros(1, dtype=torch.long, device=dev)
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    def _install(self) -> None:
        for layer, (ctx, ssm) in zip(self.model.layers, self.caches):
            layer.ssm._conv_context, layer.ssm._ssm_hiddens = ctx, ssm

    def _body(self) -> None:
        logits = self.model.step(self.token)
        if self.temperature != 1.0:
            logits = logits / self.temperature
        probs = torch.softmax(logits, dim=-1)
        if _dec.pick_supported(probs):
            # argmax, token, tokens[:, pos] and pos += 1 in one launch
            _dec.pick(probs, self.token, self.tokens, self.pos)
            return
        nxt = probs.argmax(dim=-1)
        self.token.copy_(nxt)
        self.tokens.index_copy_(1, self.pos.clamp(max=self.tokens.shape[1] - 1), nxt[:, None])
        self.pos.add_(1)

    def capture(self) -> None:
        """Warm up and capture the step (the caches' contents are overwritten
        by the next prefill)."""
        if self.graph is not None:
            return
        self._install()
        with torch.no_grad():
            side = torch.cuda.Stream(self.device)
            side.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(side):
                for _ in range(2):
                    self._body()
            torch.cuda.current_stream(self.device).wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._body()
            self.graph = graph

    def prefill(self, input_ids: torch.Tensor, lengths: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Run the prompt, fill the caches and pick the first new token (stored
        as generated token 0).  Returns the logits at position lengths - 1,
        (batch, vocab): the LM head runs on those rows only."""
        self._install()
        with torch.no_grad():
            if lengths is None:
                lengths = (input_ids != self.model.config.pad_token_id).sum(dim=1)
            last = self.model.forward_last(input_ids, lengths, use_cache=True)
            first = _greedy_pick(last, self.temperature)
            self.token.copy_(first)
            self.tokens[:, 0] = first
            self.pos.fill_(1)
        return last

    def replay(self, steps: int) -> None:
        """Advance ``steps`` tokens (one model step each)."""
        if self.graph is None:
            self.capture()
        self._install()
        for _ in range(steps):
            self.graph.replay()

    def generate(self, input_ids: torch.Tensor, check_every: int = 16) -> torch.Tensor:
        """New tokens (batch, k) of the reference's greedy loop: k is the first
        count at which every row has produced EOS, else max_new_tokens."""
        self.capture()
        self.prefill(input_ids)
        eos = self.model.config.eos_token_id
        done = 1
        while True:
            seen = (self.tokens[:, :done] == eos).any(dim=1)
            if bool(seen.all()):
                # the first count at which every row has an EOS
                first = torch.where(self.tokens[:, :done] == eos,
                                    torch.arange(done, device=self.device),
                                    torch.full_like(self.tokens[:, :done], done))
                k = int(first.min(dim=1).values.max()) + 1
                return self.tokens[:, :k].clone()
            if done >= self.max_new:
                return self.tokens[:, :self.max_new].clone()
            n = min(check_every, self.max_new - done)
            self.replay(n)
            _dec.layers_check(self.model)
            done += n
