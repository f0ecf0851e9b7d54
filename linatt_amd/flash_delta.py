"""SPD delta rule (DeltaKata) forward on MI355X: a drop-in for the forward of
``kata.spd.flash_delta`` (``kata/spd/flash_delta.py``), the mixer's
``use_delta`` branch (``kata/layer.py:377-420``).

With ``s = sqrt(scale)`` on q and k (``scale`` defaults to ``1 / E``,
``E = D / M``) and the sum-SPD kernel ``kappa(a, b) = sum_{g,h} (s a_g . s b_h)^2``:

    A_kk = kappa(k, k),  U = (I + diag(beta) strict_lower(A_kk))^-1 diag(beta) V
    num  = lower(kappa(q, k)) U,  den_t = sum_{s<=t} kappa(q_t, k_s)
    o    = num / (den + eps) if normalize else num          (float32)

* ``flash_delta(q, k, v, beta, M, scale=None, C=64, normalize=False, eps=1e-5)``
  (``flash_delta.py:1111-1116``): time-major ``(B, T, H, D)`` inputs, float32
  ``(B, T, H, DV)`` output.  The forward runs in ``liblinatt_hip.so``
  (``linatt_dkata_fwd``): a chunk-parallel solve of the 64-token diagonal
  blocks, a chunk-sequential MFMA pass for ``U`` and the KATA sum-score
  forward for the readout.  The backward (``linatt_dkata_bwd``) runs the
  KATA sum-score backward for the readout and for the erase terms around a
  reverse chunk solve, in bfloat16: with a gradient, float16 inputs run
  forward and backward in bfloat16 (float16's range cannot hold the
  backward's intermediates at small scales) and get float16 gradients.
* ``flash_delta_U`` (``:186-212``), ``flash_delta_readout`` (``:975-985``) and
  ``flash_delta_den`` (``:1049-1057``) return the forward's intermediates
  with the reference's signatures.

``C``, ``warps`` and ``BM`` are the reference's Triton tile knobs: accepted
and ignored (the HIP kernels use 64-token chunks).  Unsupported shapes raise.
"""

from __future__ import annotations

import torch

from . import _lib
from .parallel_kata_attn import _fwd as _kata_fwd

_lib.load()

__all__ = ["flash_delta", "flash_delta_U", "flash_delta_readout", "flash_delta_den"]


def _scale(D, M, scale):
    return 1.0 / (D // M) if scale is None else float(scale)


def _run(q, k, v, beta, M, scale, normalize, eps, want_U, train=False):
    _lib.require_device(q, k, v, beta)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v must share a dtype")
    if q.dim() != 4 or k.shape != q.shape or v.shape[:3] != q.shape[:3]:
        raise ValueError(f"q, k must be (B, T, H, D) and v (B, T, H, DV); got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    B, T, H, D = q.shape
    DV = v.shape[-1]
    if beta.shape != (B, T, H):
        raise ValueError(f"beta must be (B, T, H) = {(B, T, H)}, got {tuple(beta.shape)}")
    if D % M:
        raise ValueError(f"D={D} not divisible by M={M}")
    L = _lib.load()
    dt = _lib.dtype_code(q.dtype)
    if not L.linatt_dkata_supported(dt, D, DV, M):
        raise NotImplementedError(
            f"linatt_amd flash_delta: no kernel for {q.dtype}, D={D}, DV={DV}, M={M}")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    beta = beta.float().contiguous()
    # training keeps no float32 U: the backward reads the workspace's 16-bit
    # copy of U
    U = torch.empty(B, T, H, DV, device=q.device, dtype=torch.float32) if want_U else None
    o = torch.empty(B, T, H, DV, device=q.device, dtype=torch.float32)
    den = torch.empty(B, T, H, device=q.device, dtype=torch.float32)
    ws = torch.empty(L.linatt_dkata_workspace_bytes(B, T, H, D, DV, dt), device=q.device,
                     dtype=torch.uint8)
    fn = "linatt_dkata_fwd_train" if train else "linatt_dkata_fwd"
    _lib.check(fn, getattr(L, fn)(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(beta), _lib.ptr(U), _lib.ptr(o),
        _lib.ptr(den), _lib.ptr(ws), B, T, H, D, DV, M, _scale(D, M, scale),
        1 if normalize else 0, float(eps), dt, _lib.stream_of(q)))
    if train:
        return o, U, den, ws, (q, k, v, beta)
    return o, U, den


class _FlashDelta(torch.autograd.Function):
    """``_FlashDelta`` (``kata/spd/flash_delta.py:1060-1108``): the forward keeps
    the output, den and its workspace (which holds a 16-bit copy of U, all the
    backward reads of U) for the backward (``linatt_dkata_fwd_train`` /
    ``linatt_dkata_bwd``)."""

    @staticmethod
    def forward(ctx, q, k, v, beta, M, scale, normalize, eps):
        train = any(ctx.needs_input_grad[:4])
        if not train:
            o, _, _ = _run(q, k, v, beta, M, scale, normalize, eps, False)
            return o
        ctx.dtypes = (q.dtype, k.dtype, v.dtype, beta.dtype)
        if q.dtype == torch.float16 and k.dtype == v.dtype == torch.float16:
            # the backward's 16-bit intermediates (dU ~ scale^2) fall below
            # float16's normal range at small scales: with a gradient, float16
            # inputs run forward and backward in bfloat16, and the gradients
            # come back in float16
            q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
        elif q.dtype != torch.bfloat16:
            raise NotImplementedError(
                "linatt_amd flash_delta: the backward runs in bfloat16 (float16 inputs are "
                f"converted); got {q.dtype}")
        o, U, den, ws, (qc, kc, vc, bc) = _run(q, k, v, beta, M, scale, normalize, eps, False,
                                                train=True)
        # o is read back only when normalize (its z = <do', o> term)
        ctx.save_for_backward(qc, kc, vc, bc, U, o if normalize else None, den, ws)
        ctx.M, ctx.scale, ctx.normalize, ctx.eps = M, scale, normalize, eps
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, beta, U, o, den, ws = ctx.saved_tensors
        B, T, H, D = q.shape
        DV = v.shape[-1]
        M = ctx.M
        L = _lib.load()
        dt = _lib.dtype_code(q.dtype)
        do = do.float().contiguous()
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        dbeta = torch.empty(B, T, H, device=q.device, dtype=torch.float32)
        bws = torch.empty(L.linatt_dkata_bwd_workspace_bytes(B, T, H, D, DV, dt),
                          device=q.device, dtype=torch.uint8)
        _lib.check("linatt_dkata_bwd", L.linatt_dkata_bwd(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(beta), _lib.ptr(U),
            _lib.ptr(o if ctx.normalize else None), _lib.ptr(den), _lib.ptr(do), _lib.ptr(dq),
            _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dbeta), _lib.ptr(ws), _lib.ptr(bws),
            B, T, H, D, DV, M, _scale(D, M, ctx.scale), 1 if ctx.normalize else 0,
            float(ctx.eps), dt, _lib.stream_of(q)))
        tq, tk, tv, tb = ctx.dtypes
        return dq.to(tq), dk.to(tk), dv.to(tv), dbeta.to(tb), None, None, None, None


def flash_delta(q, k, v, beta, M, scale=None, C=64, normalize=False, eps=1e-5):
    """SPD delta-rule attention, float32 ``(B, T, H, DV)``
    (``kata/spd/flash_delta.py:1111-1116``)."""
    return _FlashDelta.apply(q, k, v, beta, M, scale, normalize, eps)


def flash_delta_U(q, k, v, beta, M, scale=None, C=64, warps=4):
    """Pseudo-values ``U = (I + diag(beta) strict_lower(A_kk))^-1 diag(beta) V``,
    float32 ``(B, T, H, DV)`` (``kata/spd/flash_delta.py:186-212``)."""
    _, U, _ = _run(q, k, v, beta, M, scale, False, 0.0, True)
    return U


def flash_delta_den(q, k, M, scale=None, C=64, BM=128):
    """``den_t = sum_{s<=t} kappa(q_t, k_s)``, float32 ``(B, T, H)``
    (``kata/spd/flash_delta.py:1049-1057``), from the KATA sum-score forward
    (``linatt_kata_fwd``), whose ``den`` is this sum."""
    D = q.shape[-1]
    v = torch.zeros(*k.shape[:3], 64, device=k.device, dtype=k.dtype)
    _, den = _kata_fwd(q, k, v, M, _scale(D, M, scale), "sum")
    return den


def flash_delta_readout(q, k, U, M, scale=None, C=64, BM=128):
    """``num = lower(kappa(q, k)) U``, float32 ``(B, T, H, DV)``
    (``kata/spd/flash_delta.py:975-985``): the KATA sum-score forward of
    ``(q, k, U)`` with its float32 accumulator written out
    (``linatt_kata_fwd_num``).  ``U`` is rounded to q's dtype for the
    product, as the reference's kernel loads it."""
    _lib.require_device(q, k, U)
    B, T, H, D = q.shape
    DV = U.shape[-1]
    qc, kc = q.contiguous(), k.to(q.dtype).contiguous()
    Uc = U.to(q.dtype).contiguous()
    num = torch.empty(B, T, H, DV, device=q.device, dtype=torch.float32)
    den = torch.empty(B, T, H, device=q.device, dtype=torch.float32)
    L = _lib.load()
    _lib.check("linatt_kata_fwd_num", L.linatt_kata_fwd_num(
        _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(Uc), _lib.ptr(num), _lib.ptr(den), B, T, H, H, D, DV,
        M, _scale(D, M, scale), _lib.LINATT_KATA_SUM, _lib.dtype_code(q.dtype),
        _lib.stream_of(q)))
    return num
