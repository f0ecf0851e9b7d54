"""Chunked (gated) delta rule on MI355X: drop-in for the two fla ops the
reference's DeltaNet / GatedDeltaNet baselines call.

The reference reaches this arithmetic through the third-party package
``flash-linear-attention==0.5.0`` (pinned at ``scripts/setup.sh:27``), whose
layers are selected by ``model_type: delta_net`` / ``gated_deltanet``
(``configs/model/200m/delta_net_200m.yaml:3``,
``configs/model/200m/gated_deltanet_200m.yaml:4``).  This module keeps fla's
public signatures:

* ``chunk_delta_rule(q, k, v, beta, scale=None, initial_state=None,
  output_final_state=False, cu_seqlens=None, use_qk_l2norm_in_kernel=False)``
* ``chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None,
  output_final_state=False, cu_seqlens=None, use_qk_l2norm_in_kernel=False)``

both returning ``(o, final_state)``.  Layout is fla's default time-major
``(B, T, H, D)``; states are ``(B, H, K, V)`` float32; ``scale=None`` means
``1/sqrt(K)``; ``g`` is the per-token log decay (``<= 0``).  Gradients come
back in each input's dtype.  Every computation runs in ``liblinatt_hip.so``
(``linatt_delta_fwd`` / ``linatt_delta_bwd``, plus ``linatt_l2norm_*`` for
``use_qk_l2norm_in_kernel``); float32 inputs raise, and so do
``head_first=True`` and any other keyword fla would accept but this build
does not implement.

Variable-length batches follow fla's convention: ``B == 1``, the N sequences
packed along T with offsets ``cu_seqlens`` ``(N + 1,)``, ``initial_state``
and the final state ``(N, H, K, V)``.  The sequences are laid out as the N
rows of a right-padded batch (on the GPU, by one index copy) and run through
the same kernels: the padding has beta = 0, g = 0 and zero q, k, v, so the
state passes through it unchanged, the final state of each row is that
sequence's own, and nothing flows back from it.
"""

from __future__ import annotations

import math

import torch

from . import _lib

_lib.load()  # fail at import when the HIP library is missing

__all__ = ["chunk_delta_rule", "chunk_gated_delta_rule", "l2norm"]


def _check_inputs(q, k, v, beta, g):
    _lib.require_device(q, k, v, beta, g)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, v must share a dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"linatt_amd delta rule: dtype {q.dtype} has no kernel (bf16, fp16)")
    B, T, H, K = q.shape
    if k.shape != (B, T, H, K):
        raise ValueError(f"k shape {tuple(k.shape)} != q shape {(B, T, H, K)}")
    if v.shape[:3] != (B, T, H):
        raise ValueError(f"v shape {tuple(v.shape)} does not match (B, T, H) = {(B, T, H)}")
    if beta.shape != (B, T, H):
        raise ValueError(f"beta must be (B, T, H) = {(B, T, H)}, got {tuple(beta.shape)}")
    if g is not None and g.shape != (B, T, H):
        raise ValueError(f"g must be (B, T, H) = {(B, T, H)}, got {tuple(g.shape)}")
    L = _lib.load()
    if not L.linatt_delta_supported(_lib.dtype_code(q.dtype), K, v.shape[-1]):
        raise NotImplementedError(
            f"linatt_amd delta rule: no kernel for dk={K}, dv={v.shape[-1]}, {q.dtype}")


class _L2Norm(torch.autograd.Function):
    """Row L2 normalisation ``x / sqrt(sum x^2 + eps)`` on the HIP kernels
    (the form fla applies for ``use_qk_l2norm_in_kernel=True``)."""

    @staticmethod
    def forward(ctx, x, eps):
        x = x.contiguous()
        y = torch.empty_like(x)
        rstd = torch.empty(x.shape[:-1], device=x.device, dtype=torch.float32)
        L = _lib.load()
        n, d = x.numel() // x.shape[-1], x.shape[-1]
        _lib.check("linatt_l2norm_fwd", L.linatt_l2norm_fwd(
            _lib.ptr(x), _lib.ptr(y), _lib.ptr(rstd), n, d, float(eps),
            _lib.dtype_code(x.dtype), _lib.stream_of(x)))
        ctx.save_for_backward(y, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        y, rstd = ctx.saved_tensors
        dy = dy.to(y.dtype).contiguous()
        dx = torch.empty_like(y)
        L = _lib.load()
        n, d = y.numel() // y.shape[-1], y.shape[-1]
        _lib.check("linatt_l2norm_bwd", L.linatt_l2norm_bwd(
            _lib.ptr(y), _lib.ptr(rstd), _lib.ptr(dy), _lib.ptr(dx), n, d,
            _lib.dtype_code(y.dtype), _lib.stream_of(y)))
        return dx, None


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Differentiable row L2 normalisation over the last dim (HIP)."""
    _lib.require_device(x)
    return _L2Norm.apply(x, eps)


class ChunkDeltaRuleFunction(torch.autograd.Function):
    """Autograd op over ``linatt_delta_fwd`` / ``linatt_delta_bwd``; ``g`` is
    ``None`` for the ungated rule."""

    @staticmethod
    def forward(ctx, q, k, v, beta, g, scale, initial_state, output_final_state):
        B, T, H, K = q.shape
        V = v.shape[-1]
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        beta_f = beta.float().contiguous()
        g_f = g.float().contiguous() if g is not None else None
        h0 = initial_state.float().contiguous() if initial_state is not None else None
        if h0 is not None and h0.shape != (B, H, K, V):
            raise ValueError(f"initial_state must be (B, H, K, V) = {(B, H, K, V)}")
        dt = _lib.dtype_code(q.dtype)
        L = _lib.load()
        o = torch.empty(B, T, H, V, device=q.device, dtype=v.dtype)
        ht = (torch.empty(B, H, K, V, device=q.device, dtype=torch.float32)
              if output_final_state else None)
        cbytes = L.linatt_delta_ctx_bytes(B, T, H, K, V, dt)
        cbuf = torch.empty(cbytes, device=q.device, dtype=torch.uint8)
        _lib.check("linatt_delta_fwd", L.linatt_delta_fwd(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(beta_f), _lib.ptr(g_f), _lib.ptr(h0),
            _lib.ptr(o), _lib.ptr(ht), _lib.ptr(cbuf), B, T, H, K, V, float(scale), dt,
            _lib.stream_of(q)))
        ctx.save_for_backward(q, k, v, beta_f, g_f, h0, cbuf)
        ctx.scale = scale
        ctx.dtypes = (beta.dtype, g.dtype if g is not None else None,
                      initial_state.dtype if initial_state is not None else None)
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, beta_f, g_f, h0, cbuf = ctx.saved_tensors
        B, T, H, K = q.shape
        V = v.shape[-1]
        dt = _lib.dtype_code(q.dtype)
        L = _lib.load()
        do = do.to(v.dtype).contiguous()
        dht = dht.float().contiguous() if dht is not None else None
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        dbeta = torch.empty(B, T, H, device=q.device, dtype=torch.float32)
        dg = torch.empty_like(dbeta) if g_f is not None else None
        dh0 = torch.empty_like(h0) if h0 is not None else None
        ws = torch.empty(L.linatt_delta_bwd_workspace_bytes(B, T, H, K, V, dt),
                         device=q.device, dtype=torch.uint8)
        _lib.check("linatt_delta_bwd", L.linatt_delta_bwd(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(beta_f), _lib.ptr(g_f), _lib.ptr(h0),
            _lib.ptr(do), _lib.ptr(dht), _lib.ptr(cbuf), _lib.ptr(ws), _lib.ptr(dq), _lib.ptr(dk),
            _lib.ptr(dv), _lib.ptr(dbeta), _lib.ptr(dg), _lib.ptr(dh0), B, T, H, K, V,
            float(ctx.scale), dt, _lib.stream_of(q)))
        bdt, gdt, hdt = ctx.dtypes
        return (dq, dk, dv, dbeta.to(bdt), dg.to(gdt) if dg is not None else None, None,
                dh0.to(hdt) if dh0 is not None else None, None)


def _check_kwargs(fn, kwargs):
    """fla's ops take ``**kwargs`` for deprecated arguments; the only one with
    a meaning here is ``head_first`` (a ``(B, H, T, D)`` layout), which is
    refused, as is anything unknown, so that no argument is silently lost."""
    kwargs = dict(kwargs)
    if kwargs.pop("head_first", False):
        raise NotImplementedError(
            f"{fn}: head_first=True is not supported; pass time-major (B, T, H, D) tensors")
    if kwargs:
        raise TypeError(f"{fn}: unexpected keyword arguments {sorted(kwargs)}")


def _seq_layout(cu_seqlens, T, device):
    """Row-major positions in the padded ``(N, Tmax)`` batch of the T packed
    tokens, from fla-style offsets ``cu_seqlens`` ``(N + 1,)``."""
    cu = torch.as_tensor(cu_seqlens).to("cpu", torch.int64)
    if cu.dim() != 1 or cu.numel() < 2:
        raise ValueError("cu_seqlens must be a 1-D tensor of N + 1 offsets")
    lens = cu[1:] - cu[:-1]
    if int(cu[0]) != 0 or int(cu[-1]) != T or bool((lens < 0).any()):
        raise ValueError(f"cu_seqlens must rise from 0 to T = {T}, got {cu.tolist()}")
    N, Tmax = lens.numel(), int(lens.max())
    if Tmax == 0:
        raise ValueError("cu_seqlens describes only empty sequences")
    seq = torch.repeat_interleave(torch.arange(N), lens)
    dst = seq * Tmax + torch.arange(T) - cu[:-1][seq]
    return dst.to(device), N, Tmax


def _run_varlen(q, k, v, beta, g, scale, initial_state, output_final_state, cu_seqlens):
    B, T, H, K = q.shape
    if B != 1:
        raise ValueError(f"cu_seqlens needs the sequences packed into B = 1, got B = {B}")
    dst, N, Tmax = _seq_layout(cu_seqlens, T, q.device)
    if initial_state is not None and initial_state.shape[0] != N:
        raise ValueError(f"initial_state must hold N = {N} states, got {tuple(initial_state.shape)}")

    def pad(x):  # (1, T, ...) -> (N, Tmax, ...), zeros in the padding
        z = x.new_zeros((N * Tmax,) + tuple(x.shape[2:]))
        return z.index_copy(0, dst, x[0]).reshape((N, Tmax) + tuple(x.shape[2:]))

    o, ht = ChunkDeltaRuleFunction.apply(pad(q), pad(k), pad(v), pad(beta),
                                         pad(g) if g is not None else None, scale,
                                         initial_state, output_final_state)
    o = o.reshape((N * Tmax,) + tuple(o.shape[2:])).index_select(0, dst).unsqueeze(0)
    return o, ht


def _run(q, k, v, beta, g, scale, initial_state, output_final_state, cu_seqlens,
         use_qk_l2norm_in_kernel):
    _check_inputs(q, k, v, beta, g)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if use_qk_l2norm_in_kernel:
        q, k = l2norm(q), l2norm(k)
    if cu_seqlens is not None:
        return _run_varlen(q, k, v, beta, g, scale, initial_state, output_final_state,
                           cu_seqlens)
    return ChunkDeltaRuleFunction.apply(q, k, v, beta, g, scale, initial_state,
                                        output_final_state)


def chunk_delta_rule(q, k, v, beta, scale=None, initial_state=None, output_final_state=False,
                     cu_seqlens=None, use_qk_l2norm_in_kernel=False, **kwargs):
    """DeltaNet: ``S_t = S_{t-1} + beta_t k_t (v_t - S_{t-1}^T k_t)^T``,
    ``o_t = scale S_t^T q_t``.  Returns ``(o, final_state or None)``."""
    _check_kwargs("chunk_delta_rule", kwargs)
    return _run(q, k, v, beta, None, scale, initial_state, output_final_state, cu_seqlens,
                use_qk_l2norm_in_kernel)


def chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None,
                           output_final_state=False, cu_seqlens=None,
                           use_qk_l2norm_in_kernel=False, **kwargs):
    """GatedDeltaNet: ``S_t = e^{g_t} S_{t-1} + beta_t k_t (v_t - e^{g_t}
    S_{t-1}^T k_t)^T``, ``o_t = scale S_t^T q_t``.  Returns ``(o, final_state
    or None)``."""
    _check_kwargs("chunk_gated_delta_rule", kwargs)
    return _run(q, k, v, beta, g, scale, initial_state, output_final_state, cu_seqlens,
                use_qk_l2norm_in_kernel)
