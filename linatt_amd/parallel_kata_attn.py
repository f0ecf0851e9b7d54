"""KATA-SPD parallel (flash-style) attention on MI355X: drop-in for the
reference module ``kata/parallel_kata_attn.py``.

Same public names, signatures, defaults and conventions as the reference
(``kata/layer.py:29-35`` imports ``parallel_kata_attn``,
``parallel_kata_attn_decay``, ``parallel_kata_attn_fwd``,
``parallel_kata_attn_sum`` and ``parallel_kata_attn_sum_fwd_impl`` by name):

* inputs time-major ``(B, T, H, D)``, made contiguous; GQA when
  ``HQ = G * H``;
* ``scale=None`` means ``1/sqrt(dk // num_groups)``
  (``kata/parallel_kata_attn.py:152-153``);
* ``o`` in ``v.dtype``, ``den`` float32; gradients in each input's dtype and
  ``None`` for the non-tensor arguments;
* ``bT``/``bK`` are accepted and ignored (the reference autotunes them);
  ``use_triton_bwd`` is accepted and ignored: the backward always runs the
  HIP kernels, which also cover GQA and every compiled ``num_groups``, cases
  where the reference falls back to its O(T^2)-memory PyTorch backward
  (``kata/parallel_kata_attn.py:169, 379-382``).

Every computation runs in ``liblinatt_hip.so`` (C ABI, ``include/linatt_hip.h``);
unsupported combinations raise, nothing falls back to PyTorch math.
"""

from __future__ import annotations

import math

import torch

from . import _lib

_lib.load()  # fail at import when the HIP library is missing

__all__ = [
    "parallel_kata_attn",
    "parallel_kata_attn_fwd",
    "parallel_kata_attn_fwd_impl",
    "parallel_kata_attn_bwd",
    "parallel_kata_attn_sum",
    "parallel_kata_attn_sum_fwd_impl",
    "parallel_kata_attn_bwd_sum",
    "parallel_kata_attn_decay",
    "parallel_kata_attn_onorm",
    "ParallelKataAttnFunction",
    "ParallelKataAttnSumFunction",
]

_VARIANT = {"concat": _lib.LINATT_KATA_CONCAT, "sum": _lib.LINATT_KATA_SUM}


def _default_scale(dk: int, num_groups: int) -> float:
    return 1.0 / math.sqrt(dk // num_groups)


def _prep(q, k, v):
    """Contiguous inputs sharing v's dtype; shape checks as the reference
    (``kata/parallel_kata_attn.py:229-238``)."""
    _lib.require_device(q, k, v)
    dt = v.dtype
    q = q.to(dt).contiguous()
    k = k.to(dt).contiguous()
    v = v.contiguous()
    B, T, HQ, dk = q.shape
    H = k.shape[2]
    assert k.shape[:2] == (B, T) and v.shape[:2] == (B, T), "q, k, v must share (B, T)"
    assert k.shape[-1] == dk and v.shape[2] == H, "k/v head layout mismatch"
    assert HQ % H == 0, "GQA requires HQ multiple of H"
    return q, k, v


def _fwd(q, k, v, num_groups, scale, variant, c=None):
    q, k, v = _prep(q, k, v)
    B, T, HQ, dk = q.shape
    H, dv = k.shape[2], v.shape[-1]
    assert dk % num_groups == 0, f"d_k={dk} not divisible by M={num_groups}"
    if scale is None:
        scale = _default_scale(dk, num_groups)
    o = torch.empty(B, T, HQ, dv, device=q.device, dtype=v.dtype)
    den = torch.empty(B, T, HQ, device=q.device, dtype=torch.float32)
    if c is not None:
        _lib.require_device(c)
        c = c.float().contiguous()
        assert c.shape == (B, T, HQ), f"c must be (B,T,HQ) = {(B, T, HQ)}, got {tuple(c.shape)}"
    L = _lib.load()
    _lib.check("linatt_kata_fwd", L.linatt_kata_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(c), _lib.ptr(o), _lib.ptr(den),
        B, T, HQ, H, dk, dv, num_groups, float(scale), _VARIANT[variant],
        _lib.dtype_code(v.dtype), _lib.stream_of(q)))
    return o, den


def _bwd(q, k, v, o, den, do, num_groups, scale, variant):
    q, k, v = _prep(q, k, v)
    do = do.to(v.dtype).contiguous()
    o = o.contiguous()
    den = den.float().contiguous()
    B, T, HQ, dk = q.shape
    H, dv = k.shape[2], v.shape[-1]
    dq = torch.empty_like(q)
    dk_ = torch.empty_like(k)
    dv_ = torch.empty_like(v)
    L = _lib.load()
    ws = torch.empty(L.linatt_kata_bwd_workspace_bytes(B, T, HQ, dv, _lib.dtype_code(v.dtype)) // 4,
                     device=q.device, dtype=torch.float32)
    _lib.check("linatt_kata_bwd", L.linatt_kata_bwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(den), _lib.ptr(do),
        _lib.ptr(dq), _lib.ptr(dk_), _lib.ptr(dv_), _lib.ptr(ws),
        B, T, HQ, H, dk, dv, num_groups, float(scale), _VARIANT[variant],
        _lib.dtype_code(v.dtype), _lib.stream_of(q)))
    return dq, dk_, dv_


def parallel_kata_attn_fwd_impl(q, k, v, num_groups, scale, bT, bK, c=None):
    """Concat-SPD causal forward; returns ``(o, den)``
    (reference ``kata/parallel_kata_attn.py:211-288``).  ``c`` is an optional
    ``(B, T, HQ)`` float32 cumulative log-decay: scores are multiplied by
    ``exp(min(c_t - c_s, 0))``."""
    return _fwd(q, k, v, num_groups, scale, "concat", c)


def parallel_kata_attn_fwd(q, k, v, num_groups=4, scale=None, bT=64, bK=64):
    """No-autograd forward returning ``(o, den)``
    (reference ``kata/parallel_kata_attn.py:357-361``)."""
    if scale is None:
        scale = _default_scale(q.shape[-1], num_groups)
    return parallel_kata_attn_fwd_impl(q, k, v, num_groups, scale, bT, bK)


def parallel_kata_attn_bwd(q, k, v, o, den, do, num_groups, scale, bT=64, bK=64):
    """Concat-SPD backward ``(dq, dk, dv)``; same signature and result as the
    reference ``parallel_kata_attn_bwd`` (``kata/parallel_kata_attn.py:49-146``)
    and ``parallel_kata_attn_bwd_triton`` (``:364-529``), on the HIP kernels."""
    return _bwd(q, k, v, o, den, do, num_groups, scale, "concat")


parallel_kata_attn_bwd_triton = parallel_kata_attn_bwd


class ParallelKataAttnFunction(torch.autograd.Function):
    """Reference ``kata/parallel_kata_attn.py:149-195``."""

    @staticmethod
    def forward(ctx, q, k, v, num_groups, scale, bT, bK, use_triton_bwd):
        if scale is None:
            scale = _default_scale(q.shape[-1], num_groups)
        o, den = parallel_kata_attn_fwd_impl(q, k, v, num_groups, scale, bT, bK)
        ctx.save_for_backward(q, k, v, o, den)
        ctx.num_groups = num_groups
        ctx.scale = scale
        ctx.dtypes = (q.dtype, k.dtype, v.dtype)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, den = ctx.saved_tensors
        dq, dk, dv = parallel_kata_attn_bwd(q, k, v, o, den, do, ctx.num_groups, ctx.scale)
        qd, kd, vd = ctx.dtypes
        return dq.to(qd), dk.to(kd), dv.to(vd), None, None, None, None, None


def parallel_kata_attn(q, k, v, num_groups=4, scale=None, bT=64, bK=64, use_triton_bwd=True):
    """Autograd concat-SPD attention (reference ``kata/parallel_kata_attn.py:198-208``)."""
    return ParallelKataAttnFunction.apply(q, k, v, num_groups, scale, bT, bK, use_triton_bwd)


# ---------------------------------------------------------------------------
# Sum-SPD score: A = sum_{i,j} (scale q_i . k_j)^2
# ---------------------------------------------------------------------------


def parallel_kata_attn_sum_fwd_impl(q, k, v, num_groups, scale, bT, bK):
    """Sum-SPD causal forward ``(o, den)``
    (reference ``kata/parallel_kata_attn.py:539-576``)."""
    return _fwd(q, k, v, num_groups, scale, "sum")


def parallel_kata_attn_bwd_sum(q, k, v, o, den, do, num_groups, scale):
    """Sum-SPD backward ``(dq, dk, dv)``; result of the reference's
    ``parallel_kata_attn_bwd_sum_torch`` (``kata/parallel_kata_attn.py:579-653``)
    and ``parallel_kata_attn_sum_bwd_triton_M{2,4}`` (``:755-901``)."""
    return _bwd(q, k, v, o, den, do, num_groups, scale, "sum")


parallel_kata_attn_bwd_sum_torch = parallel_kata_attn_bwd_sum


class ParallelKataAttnSumFunction(torch.autograd.Function):
    """Reference ``kata/parallel_kata_attn.py:656-734``."""

    @staticmethod
    def forward(ctx, q, k, v, num_groups, scale, bT, bK, use_triton_bwd):
        if scale is None:
            scale = _default_scale(q.shape[-1], num_groups)
        o, den = parallel_kata_attn_sum_fwd_impl(q, k, v, num_groups, scale, bT, bK)
        ctx.save_for_backward(q, k, v, o, den)
        ctx.num_groups = num_groups
        ctx.scale = scale
        ctx.dtypes = (q.dtype, k.dtype, v.dtype)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, den = ctx.saved_tensors
        dq, dk, dv = parallel_kata_attn_bwd_sum(q, k, v, o, den, do, ctx.num_groups, ctx.scale)
        qd, kd, vd = ctx.dtypes
        return dq.to(qd), dk.to(kd), dv.to(vd), None, None, None, None, None


def parallel_kata_attn_sum(q, k, v, num_groups=4, scale=None, bT=64, bK=64, use_triton_bwd=True):
    """Autograd sum-SPD attention (reference ``kata/parallel_kata_attn.py:737-752``)."""
    return ParallelKataAttnSumFunction.apply(q, k, v, num_groups, scale, bT, bK, use_triton_bwd)


# ---------------------------------------------------------------------------
# Decayed concat score: A * exp(min(c_t - c_s, 0))
# ---------------------------------------------------------------------------


class _KataDecayFunction(torch.autograd.Function):
    """Reference ``kata/parallel_kata_attn.py:313-347``: forward and backward
    (dq, dk, dv and dc) on the HIP kernels (``linatt_kata_fwd`` with ``c``,
    ``linatt_kata_bwd_decay``), without the reference's O(T^2)-memory
    autograd recompute."""

    @staticmethod
    def forward(ctx, q, k, v, c, num_groups, scale):
        if scale is None:
            scale = _default_scale(q.shape[-1], num_groups)
        o, den = parallel_kata_attn_fwd_impl(q, k, v, num_groups, scale, 64, 64, c=c)
        ctx.save_for_backward(q, k, v, c, o, den)
        ctx.num_groups, ctx.scale = num_groups, scale
        ctx.dtypes = (q.dtype, k.dtype, v.dtype, c.dtype)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, c, o, den = ctx.saved_tensors
        qc, kc, vc = _prep(q, k, v)
        cf = c.float().contiguous()
        do = do.to(vc.dtype).contiguous()
        B, T, HQ, dk = qc.shape
        H, dv = kc.shape[2], vc.shape[-1]
        dq, dk_, dv_ = torch.empty_like(qc), torch.empty_like(kc), torch.empty_like(vc)
        dc = torch.empty_like(cf)
        # bound to locals: a temporary made inside the argument list would be
        # freed (and its memory reusable) before the kernels read it
        oc = o.contiguous()
        denc = den.float().contiguous()
        L = _lib.load()
        ws = torch.empty(L.linatt_kata_bwd_workspace_bytes(B, T, HQ, dv, _lib.dtype_code(vc.dtype)) // 4,
                         device=q.device, dtype=torch.float32)
        _lib.check("linatt_kata_bwd_decay", L.linatt_kata_bwd_decay(
            _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.ptr(cf), _lib.ptr(oc),
            _lib.ptr(denc), _lib.ptr(do), _lib.ptr(dq), _lib.ptr(dk_),
            _lib.ptr(dv_), _lib.ptr(dc), _lib.ptr(ws), B, T, HQ, H, dk, dv, ctx.num_groups,
            float(ctx.scale), _lib.dtype_code(vc.dtype), _lib.stream_of(qc)))
        qd, kd, vd, cd = ctx.dtypes
        return dq.to(qd), dk_.to(kd), dv_.to(vd), dc.to(cd), None, None


def parallel_kata_attn_decay(q, k, v, c, num_groups=2, scale=None):
    """Decayed SPD attention (reference ``kata/parallel_kata_attn.py:350-354``):
    ``o_t = sum_{s<=t} exp(min(c_t-c_s,0)) A[t,s] v_s / sum(...)``."""
    return _KataDecayFunction.apply(q, k, v, c, num_groups, scale)


# ---------------------------------------------------------------------------
# The mixer's output RMSNorm fused into the attention kernels
# ---------------------------------------------------------------------------


def _onorm_fused(dtype, dk, dv, need_grad):
    """The fused kernels cover dk = dv = 64 in bf16 (and fp16 without a
    gradient: the fp16 dk/dv pass reads the unscaled dO, which the fused dq
    pass never forms)."""
    if dk != 64 or dv != 64:
        return False
    return dtype == torch.bfloat16 or (dtype == torch.float16 and not need_grad)


class _KataONormFunction(torch.autograd.Function):
    """y = RMSNorm(KATA(q, k, v)) per (b, t, head) row: ``linatt_kata_fwd_onorm``
    writes o, den, y and rstd in one forward; ``linatt_kata_bwd_onorm`` forms
    the norm's dO from dy inside the dq pass and sums the weight gradient."""

    @staticmethod
    def forward(ctx, q, k, v, c, weight, eps, num_groups, scale, variant):
        qc, kc, vc = _prep(q, k, v)
        B, T, HQ, dk = qc.shape
        H, dv = kc.shape[2], vc.shape[-1]
        if scale is None:
            scale = _default_scale(dk, num_groups)
        cf = None
        if c is not None:
            _lib.require_device(c)
            cf = c.float().contiguous()
            assert cf.shape == (B, T, HQ), f"c must be (B,T,HQ) = {(B, T, HQ)}, got {tuple(cf.shape)}"
        w = None
        if weight is not None:
            _lib.require_device(weight)
            w = weight.detach().float().contiguous()
        o = torch.empty(B, T, HQ, dv, device=q.device, dtype=vc.dtype)
        y = torch.empty_like(o)
        den = torch.empty(B, T, HQ, device=q.device, dtype=torch.float32)
        rstd = torch.empty_like(den)
        L = _lib.load()
        _lib.check("linatt_kata_fwd_onorm", L.linatt_kata_fwd_onorm(
            _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.ptr(cf), _lib.ptr(o), _lib.ptr(den),
            _lib.ptr(w), float(eps), _lib.ptr(y), _lib.ptr(rstd), B, T, HQ, H, dk, dv, num_groups,
            float(scale), _VARIANT[variant], _lib.dtype_code(vc.dtype), _lib.stream_of(qc)))
        ctx.save_for_backward(qc, kc, vc, cf, o, den, rstd, w)
        ctx.args = (num_groups, float(scale), variant)
        ctx.dtypes = (q.dtype, k.dtype, v.dtype, c.dtype if c is not None else None,
                      weight.dtype if weight is not None else None)
        return y

    @staticmethod
    def backward(ctx, dy):
        q, k, v, cf, o, den, rstd, w = ctx.saved_tensors
        num_groups, scale, variant = ctx.args
        B, T, HQ, dk = q.shape
        H, dv = k.shape[2], v.shape[-1]
        dy = dy.to(v.dtype).contiguous()
        dq, dk_, dv_ = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        dc = torch.empty_like(cf) if cf is not None else None
        dw = torch.empty(dv, device=q.device, dtype=torch.float32) if w is not None else None
        L = _lib.load()
        ws = torch.empty(L.linatt_kata_bwd_onorm_workspace_bytes(B, T, HQ, dv, _lib.dtype_code(v.dtype)),
                         device=q.device, dtype=torch.uint8)
        _lib.check("linatt_kata_bwd_onorm", L.linatt_kata_bwd_onorm(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(cf), _lib.ptr(o), _lib.ptr(den),
            _lib.ptr(rstd), _lib.ptr(w), _lib.ptr(dy), _lib.ptr(dq), _lib.ptr(dk_), _lib.ptr(dv_),
            _lib.ptr(dc), _lib.ptr(dw), _lib.ptr(ws), B, T, HQ, H, dk, dv, num_groups, scale,
            _VARIANT[variant], _lib.dtype_code(v.dtype), _lib.stream_of(q)))
        qd, kd, vd, cd, wd = ctx.dtypes
        return (dq.to(qd), dk_.to(kd), dv_.to(vd), dc.to(cd) if dc is not None else None,
                dw.to(wd) if dw is not None else None, None, None, None, None)


def parallel_kata_attn_onorm(q, k, v, norm_weight=None, eps=1e-5, num_groups=4, scale=None,
                             variant="concat", c=None):
    """KATA attention followed by the mixer's output RMSNorm over each
    ``(b, t, head)`` row of o (``kata/layer.py:456-487, 539``:
    ``self.norm(parallel_kata_attn(...))`` with ``fla.modules.RMSNorm(head_v_dim,
    eps=norm_eps, dtype=float32)``).  Returns ``y (B, T, HQ, dv)`` in v's
    dtype; gradients flow to q, k, v, ``c`` (the decayed score's cumulative
    log-decay, concat only) and ``norm_weight``.

    At dk = dv = 64 in bf16 (fp16 without a gradient) the norm runs inside
    the attention kernels: the forward's epilogue normalises each row it
    writes, and the backward's dq pass forms the norm's gradient in
    registers.  Elsewhere it is the attention op followed by
    ``linatt_amd.mixer.rms_norm`` (both HIP)."""
    if variant not in _VARIANT:
        raise ValueError(f"variant must be 'concat' or 'sum', got {variant!r}")
    if c is not None and variant != "concat":
        raise NotImplementedError("decay is only defined for the concat score")
    need_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (q, k, v, c, norm_weight))
    if _onorm_fused(v.dtype, q.shape[-1], v.shape[-1], need_grad):
        return _KataONormFunction.apply(q, k, v, c, norm_weight, float(eps), num_groups, scale,
                                        variant)
    from .mixer import rms_norm
    if c is not None:
        o = parallel_kata_attn_decay(q, k, v, c, num_groups, scale)
    elif variant == "sum":
        o = parallel_kata_attn_sum(q, k, v, num_groups, scale)
    else:
        o = parallel_kata_attn(q, k, v, num_groups, scale)
    return rms_norm(o, norm_weight, eps)
