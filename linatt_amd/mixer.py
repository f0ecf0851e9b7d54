"""The KATA token mixer's non-GEMM prologue / epilogue on MI355X.

``kata/layer.py`` KataAttention.forward runs, around the attention op, the
causal short convolutions with SiLU on the projected q, k, v (``:299-318``,
modules built at ``:178-197``) and an fp32 RMSNorm over each head of the
output (``:539``, built at ``:199-205``; the q/k RMSNorm of ``:126-128, 347``
is the same op).  Both modules come from the third-party ``fla.modules``
(``ShortConvolution``, ``RMSNorm``; flash-linear-attention==0.5.0).  This
module provides drop-ins with the same constructor arguments, parameter names
and shapes (so checkpoints load) and call contract, running on
``liblinatt_hip.so``:

* ``ShortConvolution(hidden_size, kernel_size, bias=False, activation="silu")``:
  ``forward(x, cache=None, output_final_state=False)`` returns ``(y, cache)``
  with ``x, y (B, T, C)`` and the decode cache ``(B, C, W)`` holding the last
  W inputs, newest last (``linatt_short_conv_fwd`` / ``_bwd``);
* ``RMSNorm(hidden_size, elementwise_affine=True, eps=1e-5)`` over the last
  dim, fp32 arithmetic, output in the input's dtype (``linatt_rmsnorm_fwd`` /
  ``_bwd``);
* ``RotaryEmbedding(dim, base=10000.0, interleaved=False)``:
  ``forward(q, k, seqlen_offset=0)`` returns the rotated ``(q, k)``
  (``linatt_rope``; the backward is the inverse rotation).

All have autograd backwards.  ``qk_prologue`` (and ``fused_qk_prologue``,
which takes the three modules) runs the q or k chain of ``:305-372`` --
short convolution, per-head RMSNorm or L2 norm, rotary embedding -- as one
kernel pair (``linatt_qk_prologue_fwd`` / ``_bwd``), keeping the
intermediates in fp32.  The q/k/v projections and ``o_proj`` stay library
GEMMs.  Unsupported arguments (fla's ``residual``, ``mask``, ``cu_seqlens``,
a norm bias) raise.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from . import _lib

_lib.load()

__all__ = ["short_conv", "rms_norm", "rotary", "qk_prologue", "fused_qk_prologue",
           "ShortConvolution", "RMSNorm", "RotaryEmbedding"]

_ACT = {None: 0, "identity": 0, "silu": 1, "swish": 1}


def _act(activation):
    try:
        return _ACT[activation]
    except KeyError:
        raise NotImplementedError(f"linatt_amd short conv: activation {activation!r}") from None


class _ShortConvFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, cache, act, want_state):
        _lib.require_device(x, weight)
        B, T, C = x.shape
        W = weight.shape[-1]
        L = _lib.load()
        x = x.contiguous()
        w2 = weight.detach().reshape(C, W).float().contiguous()
        b = bias.detach().float().contiguous() if bias is not None else None
        if cache is not None:
            _lib.require_device(cache)
            if cache.shape != (B, C, W):
                raise ValueError(f"cache must be (B, C, W) = {(B, C, W)}, got {tuple(cache.shape)}")
            cache = cache.to(x.dtype).contiguous()
        y = torch.empty_like(x)
        state = torch.empty(B, C, W, device=x.device, dtype=x.dtype) if want_state else None
        _lib.check("linatt_short_conv_fwd", L.linatt_short_conv_fwd(
            _lib.ptr(x), _lib.ptr(w2), _lib.ptr(b), _lib.ptr(cache), _lib.ptr(y), _lib.ptr(state),
            B, T, C, W, act, _lib.dtype_code(x.dtype), _lib.stream_of(x)))
        ctx.save_for_backward(x, w2, b, cache)
        ctx.act, ctx.wshape, ctx.wdtype = act, weight.shape, weight.dtype
        ctx.has_bias = bias is not None
        ctx.bdtype = bias.dtype if bias is not None else None
        if state is not None:
            ctx.mark_non_differentiable(state)
        return y, state

    @staticmethod
    def backward(ctx, dy, _dstate):
        x, w2, b, cache = ctx.saved_tensors
        B, T, C = x.shape
        W = w2.shape[1]
        L = _lib.load()
        dy = dy.to(x.dtype).contiguous()
        dx = torch.empty_like(x)
        dw = torch.empty(C, W, device=x.device, dtype=torch.float32)
        db = torch.empty(C, device=x.device, dtype=torch.float32) if ctx.has_bias else None
        ws = torch.empty(L.linatt_short_conv_bwd_workspace_bytes(B, T, C, W), device=x.device,
                         dtype=torch.uint8)
        _lib.check("linatt_short_conv_bwd", L.linatt_short_conv_bwd(
            _lib.ptr(x), _lib.ptr(w2), _lib.ptr(b), _lib.ptr(cache), _lib.ptr(dy), _lib.ptr(dx),
            _lib.ptr(dw), _lib.ptr(db), _lib.ptr(ws), B, T, C, W, ctx.act,
            _lib.dtype_code(x.dtype), _lib.stream_of(x)))
        dw = dw.reshape(ctx.wshape).to(ctx.wdtype)
        return dx, dw, (db.to(ctx.bdtype) if db is not None else None), None, None, None


def short_conv(x, weight, bias=None, activation="silu", cache=None, output_final_state=False):
    """Causal depthwise convolution of ``x (B, T, C)`` with ``weight (C, 1, W)``
    (or ``(C, W)``), then the activation.  Returns ``(y, final_cache)``; the
    cache is ``None`` unless ``output_final_state``."""
    if x.dim() != 3:
        raise ValueError(f"x must be (B, T, C), got {tuple(x.shape)}")
    if weight.shape[0] != x.shape[-1] or weight.numel() != weight.shape[0] * weight.shape[-1]:
        raise ValueError(f"weight must be (C, 1, W) with C = {x.shape[-1]}, got {tuple(weight.shape)}")
    y, state = _ShortConvFn.apply(x, weight, bias, cache, _act(activation), bool(output_final_state))
    return y, state


class ShortConvolution(nn.Module):
    """Drop-in for ``fla.modules.ShortConvolution`` as ``kata/layer.py:178-197``
    builds it: parameters ``weight (C, 1, W)`` and optional ``bias (C)``
    (``nn.Conv1d``'s names and initialisation)."""

    def __init__(self, hidden_size, kernel_size, bias=False, activation="silu", device=None,
                 dtype=None, **kwargs):
        super().__init__()
        # fla's backend switches select among its own implementations
        for k in kwargs:
            if k not in ("use_fast_conv1d", "backend"):
                raise TypeError(f"ShortConvolution: unexpected keyword argument {k!r}")
        _act(activation)
        self.hidden_size, self.kernel_size, self.activation = hidden_size, kernel_size, activation
        fk = {"device": device, "dtype": dtype}
        self.weight = nn.Parameter(torch.empty(hidden_size, 1, kernel_size, **fk))
        self.bias = nn.Parameter(torch.empty(hidden_size, **fk)) if bias else None
        self.reset_parameters()

    def reset_parameters(self):
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            bound = 1.0 / math.sqrt(self.kernel_size)
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, x, residual=None, mask=None, cache=None, output_final_state=False,
                cu_seqlens=None, **kwargs):
        if residual is not None or mask is not None or cu_seqlens is not None or kwargs:
            raise NotImplementedError("linatt_amd ShortConvolution: residual, mask, cu_seqlens "
                                      "and other options are not supported")
        return short_conv(x, self.weight, self.bias, self.activation, cache, output_final_state)


class _RMSNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps):
        _lib.require_device(x)
        d = x.shape[-1]
        xr = x.contiguous().reshape(-1, d)
        n = xr.shape[0]
        w = weight.detach().float().contiguous() if weight is not None else None
        y = torch.empty_like(xr)
        rstd = torch.empty(n, device=x.device, dtype=torch.float32)
        L = _lib.load()
        _lib.check("linatt_rmsnorm_fwd", L.linatt_rmsnorm_fwd(
            _lib.ptr(xr), _lib.ptr(w), _lib.ptr(y), _lib.ptr(rstd), n, d, float(eps),
            _lib.dtype_code(x.dtype), _lib.stream_of(x)))
        ctx.save_for_backward(xr, w, rstd)
        ctx.shape, ctx.wdtype = x.shape, weight.dtype if weight is not None else None
        return y.reshape(x.shape)

    @staticmethod
    def backward(ctx, dy):
        xr, w, rstd = ctx.saved_tensors
        n, d = xr.shape
        L = _lib.load()
        g = dy.to(xr.dtype).contiguous().reshape(n, d)
        dx = torch.empty_like(xr)
        dw = torch.empty(d, device=xr.device, dtype=torch.float32) if w is not None else None
        ws = torch.empty(L.linatt_rmsnorm_bwd_workspace_bytes(n, d), device=xr.device,
                         dtype=torch.uint8)
        _lib.check("linatt_rmsnorm_bwd", L.linatt_rmsnorm_bwd(
            _lib.ptr(xr), _lib.ptr(w), _lib.ptr(rstd), _lib.ptr(g), _lib.ptr(dx), _lib.ptr(dw),
            _lib.ptr(ws), n, d, _lib.dtype_code(xr.dtype), _lib.stream_of(xr)))
        return dx.reshape(ctx.shape), (dw.to(ctx.wdtype) if dw is not None else None), None


def rms_norm(x, weight=None, eps=1e-5):
    """``x / sqrt(mean(x^2) + eps) * weight`` over the last dim (fp32
    arithmetic, output in x's dtype)."""
    return _RMSNormFn.apply(x, weight, eps)


class RMSNorm(nn.Module):
    """Drop-in for ``fla.modules.RMSNorm`` as ``kata/layer.py:126-128, 199-205``
    builds it (``weight (hidden_size,)``, no bias)."""

    def __init__(self, hidden_size, elementwise_affine=True, bias=False, eps=1e-5, device=None,
                 dtype=None):
        super().__init__()
        if bias:
            raise NotImplementedError("linatt_amd RMSNorm: bias is not supported")
        self.hidden_size, self.eps, self.elementwise_affine = hidden_size, eps, elementwise_affine
        self.weight = (nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))
                       if elementwise_affine else None)
        self.register_parameter("bias", None)

    def forward(self, x, residual=None, prenorm=False, residual_in_fp32=False):
        if residual is not None or prenorm:
            raise NotImplementedError("linatt_amd RMSNorm: residual / prenorm are not supported")
        if x.shape[-1] != self.hidden_size:
            raise ValueError(f"last dim {x.shape[-1]} != hidden_size {self.hidden_size}")
        return rms_norm(x, self.weight, self.eps)


class _RopeFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, rot_dim, base, offset, interleaved):
        _lib.require_device(x)
        if x.dim() != 4:
            raise ValueError(f"x must be (B, T, H, D), got {tuple(x.shape)}")
        x = x.contiguous()
        y = torch.empty_like(x)
        ctx.args = (rot_dim, base, offset, interleaved)
        _rope(x, y, rot_dim, base, offset, interleaved, False)
        return y

    @staticmethod
    def backward(ctx, dy):
        dy = dy.contiguous()
        dx = torch.empty_like(dy)
        _rope(dy, dx, *ctx.args, True)
        return dx, None, None, None, None


def _rope(x, y, rot_dim, base, offset, interleaved, inverse):
    B, T, H, D = x.shape
    L = _lib.load()
    _lib.check("linatt_rope", L.linatt_rope(
        _lib.ptr(x), _lib.ptr(y), B, T, H, D, rot_dim, float(base), int(offset),
        1 if interleaved else 0, 1 if inverse else 0, _lib.dtype_code(x.dtype),
        _lib.stream_of(x)))


def rotary(x, rot_dim=None, base=10000.0, offset=0, interleaved=False):
    """Rotary position embedding of ``x (B, T, H, D)`` over its first
    ``rot_dim`` dims (default all), positions ``offset .. offset + T - 1``."""
    return _RopeFn.apply(x, x.shape[-1] if rot_dim is None else int(rot_dim), base, offset,
                         interleaved)


class RotaryEmbedding(nn.Module):
    """Drop-in for ``fla.modules.RotaryEmbedding`` as ``kata/layer.py:130-148``
    builds it and ``:352-372`` calls it: ``forward(q, k, seqlen_offset=0,
    max_seqlen=None)`` on ``(B, T, H, D)`` tensors."""

    def __init__(self, dim, base=10000.0, scale_base=None, interleaved=False,
                 pos_idx_in_fp32=True, device=None):
        super().__init__()
        if scale_base is not None:
            raise NotImplementedError("linatt_amd RotaryEmbedding: scale_base (xPos) is not supported")
        self.dim, self.base, self.interleaved = int(dim), float(base), bool(interleaved)

    def forward(self, q, k, seqlen_offset=0, max_seqlen=None, cu_seqlens=None, **kwargs):
        if cu_seqlens is not None or kwargs or isinstance(seqlen_offset, torch.Tensor):
            raise NotImplementedError("linatt_amd RotaryEmbedding: cu_seqlens, per-sequence "
                                      "offsets and other options are not supported")
        return (rotary(q, self.dim, self.base, seqlen_offset, self.interleaved),
                rotary(k, self.dim, self.base, seqlen_offset, self.interleaved))


_NORM = {None: 0, "none": 0, "rmsnorm": 1, "l2": 2}


class _QKPrologueFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, conv_weight, conv_bias, norm_weight, cache, cfg, want_state):
        _lib.require_device(x, conv_weight)
        H, D, W, act, norm, eps, rw, rot, base, offset, inter = cfg
        B, T, C = x.shape
        L = _lib.load()
        x = x.contiguous()
        w2 = conv_weight.detach().reshape(C, W).float().contiguous()
        b = conv_bias.detach().float().contiguous() if conv_bias is not None else None
        nw = norm_weight.detach().float().contiguous() if norm_weight is not None else None
        for t in (b, nw):
            if t is not None:
                _lib.require_device(t)
        if cache is not None:
            _lib.require_device(cache)
            if cache.shape != (B, C, W):
                raise ValueError(f"cache must be (B, C, W) = {(B, C, W)}, got {tuple(cache.shape)}")
            cache = cache.to(x.dtype).contiguous()
        y = torch.empty(B, T, H, D, device=x.device, dtype=x.dtype)
        state = torch.empty(B, C, W, device=x.device, dtype=x.dtype) if want_state else None
        _lib.check("linatt_qk_prologue_fwd", L.linatt_qk_prologue_fwd(
            _lib.ptr(x), _lib.ptr(w2), _lib.ptr(b), _lib.ptr(cache), _lib.ptr(nw), _lib.ptr(y),
            _lib.ptr(state), B, T, H, D, W, act, norm, eps, rw, rot, base, offset, inter,
            _lib.dtype_code(x.dtype), _lib.stream_of(x)))
        ctx.save_for_backward(x, w2, b, nw, cache)
        ctx.cfg = cfg
        ctx.dtypes = (conv_weight.dtype, conv_bias.dtype if conv_bias is not None else None,
                      norm_weight.dtype if norm_weight is not None else None)
        ctx.wshape = conv_weight.shape
        if state is not None:
            ctx.mark_non_differentiable(state)
        return y, state

    @staticmethod
    def backward(ctx, dy, _dstate):
        x, w2, b, nw, cache = ctx.saved_tensors
        H, D, W, act, norm, eps, rw, rot, base, offset, inter = ctx.cfg
        B, T, C = x.shape
        L = _lib.load()
        dy = dy.to(x.dtype).contiguous()
        dx = torch.empty_like(x)
        dw = torch.empty(C, W, device=x.device, dtype=torch.float32)
        db = torch.empty(C, device=x.device, dtype=torch.float32) if b is not None else None
        dnw = torch.empty(D, device=x.device, dtype=torch.float32) if nw is not None else None
        ws = torch.empty(L.linatt_qk_prologue_bwd_workspace_bytes(B, T, H, D, W),
                         device=x.device, dtype=torch.uint8)
        _lib.check("linatt_qk_prologue_bwd", L.linatt_qk_prologue_bwd(
            _lib.ptr(x), _lib.ptr(w2), _lib.ptr(b), _lib.ptr(cache), _lib.ptr(nw), _lib.ptr(dy),
            _lib.ptr(dx), _lib.ptr(dw), _lib.ptr(db), _lib.ptr(dnw), _lib.ptr(ws), B, T, H, D, W,
            act, norm, eps, rw, rot, base, offset, inter, _lib.dtype_code(x.dtype),
            _lib.stream_of(x)))
        wdt, bdt, ndt = ctx.dtypes
        return (dx, dw.reshape(ctx.wshape).to(wdt), db.to(bdt) if db is not None else None,
                dnw.to(ndt) if dnw is not None else None, None, None, None)


def qk_prologue(x, conv_weight, conv_bias=None, *, head_dim, activation="silu", norm="rmsnorm",
                norm_weight=None, eps=None, rot_dim=None, rope_width=None, base=10000.0,
                offset=0, interleaved=True, cache=None, output_final_state=False):
    """The q or k prologue of ``kata/layer.py:305-372`` in one kernel:
    ``x (B, T, H * head_dim)`` (the projection output) through the causal
    short convolution + activation (``conv_weight (C, 1, W)`` or ``(C, W)``,
    ``cache`` as ``short_conv``), the per-head norm (``norm="rmsnorm"`` with
    ``norm_weight (head_dim,)`` or None, eps 1e-5 by default; ``"l2"``, fla's
    ``l2norm``, eps 1e-6 by default; ``None``) and the rotary embedding of
    rows of ``rope_width`` dims (default ``head_dim``; the group width E for
    the mixer's ``rope_group``) over their first ``rot_dim`` dims (default
    ``rope_width``; 0: no rotation) at positions ``offset ..``.  Returns
    ``(y (B, T, H, head_dim), final_cache)``; the intermediates stay in fp32,
    so y differs from the three-module chain by that chain's two roundings to
    x's dtype."""
    if x.dim() != 3:
        raise ValueError(f"x must be (B, T, H * head_dim), got {tuple(x.shape)}")
    C = x.shape[-1]
    D = int(head_dim)
    if D <= 0 or C % D:
        raise ValueError(f"the channel count {C} is not a multiple of head_dim {D}")
    if conv_weight.shape[0] != C or conv_weight.numel() != C * conv_weight.shape[-1]:
        raise ValueError(f"conv_weight must be (C, 1, W) with C = {C}, got {tuple(conv_weight.shape)}")
    if conv_bias is not None and conv_bias.shape != (C,):
        raise ValueError(f"conv_bias must be ({C},), got {tuple(conv_bias.shape)}")
    if norm not in _NORM:
        raise ValueError(f"norm must be 'rmsnorm', 'l2' or None, got {norm!r}")
    nk = _NORM[norm]
    if nk != 1 and norm_weight is not None:
        raise ValueError("norm_weight is only used with norm='rmsnorm'")
    if norm_weight is not None and norm_weight.shape != (D,):
        raise ValueError(f"norm_weight must be ({D},), got {tuple(norm_weight.shape)}")
    if eps is None:
        eps = 1e-6 if nk == 2 else 1e-5
    rw = D if rope_width is None else int(rope_width)
    rot = rw if rot_dim is None else int(rot_dim)
    if isinstance(offset, torch.Tensor):
        raise NotImplementedError("qk_prologue: per-sequence offsets are not supported")
    cfg = (C // D, D, int(conv_weight.shape[-1]), _act(activation), nk, float(eps), rw, rot,
           float(base), int(offset), 1 if interleaved else 0)
    return _QKPrologueFn.apply(x, conv_weight, conv_bias, norm_weight, cache, cfg,
                               bool(output_final_state))


def fused_qk_prologue(x, conv, norm, rotary, head_dim, seqlen_offset=0, cache=None,
                      output_final_state=False):
    """``qk_prologue`` configured from the mixer's modules: ``conv`` a
    ``ShortConvolution``; ``norm`` an ``RMSNorm`` (its weight and eps), the
    string ``"l2"`` or None; ``rotary`` a ``RotaryEmbedding`` (its dim is the
    rotation row width: the head dim, or E under ``rope_group``) or None.
    Equals ``rotary(norm(conv(x)[0].view(B, T, H, D)))`` up to the chain's
    intermediate roundings."""
    if norm is None or isinstance(norm, str):
        if norm not in (None, "l2"):
            raise ValueError(f"norm must be an RMSNorm module, 'l2' or None, got {norm!r}")
        nk, nw, eps = norm, None, None
    elif hasattr(norm, "weight") and hasattr(norm, "eps"):
        # this module's RMSNorm or fla's (weight (head_dim,) or None, eps)
        width = getattr(norm, "hidden_size", head_dim)
        if width != head_dim:
            raise ValueError(f"RMSNorm width {width} != head_dim {head_dim}")
        nk, nw, eps = "rmsnorm", norm.weight, norm.eps
    else:
        raise TypeError("norm must be an RMSNorm module (weight, eps), 'l2' or None")
    if rotary is None:
        rw, rot, base, inter = None, 0, 10000.0, True
    else:
        rw = rot = rotary.dim
        base, inter = rotary.base, rotary.interleaved
    return qk_prologue(x, conv.weight, conv.bias, head_dim=head_dim, activation=conv.activation,
                       norm=nk, norm_weight=nw, eps=eps, rot_dim=rot, rope_width=rw, base=base,
                       offset=seqlen_offset, interleaved=inter, cache=cache,
                       output_final_state=output_final_state)
