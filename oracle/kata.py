"""Float64 CPU restatement of the reference's KATA-SPD attention math.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): used by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``.
The product path in ``linatt_amd`` never imports this module.

Conventions (reference ``kata/parallel_kata_attn.py``):

* time-major tensors: q ``(B,T,HQ,dk)``, k ``(B,T,H,dk)``, v ``(B,T,H,dv)``;
  GQA when ``HQ = G*H`` (query head ``hq`` reads kv head ``hq // G``).
* ``M`` SPD groups of width ``E = dk // M``; ``scale=None`` means ``1/sqrt(E)``
  (``parallel_kata_attn.py:152-153, 241-244``).
* concat score ``A[t,s] = sum_g (scale * q_g[t].k_g[s])**2``; sum score
  ``A[t,s] = sum_{i,j} (scale * q_i[t].k_j[s])**2``; causal ``s <= t``.
* forward normalisation ``o = (A V) / den`` with ``den = sum_s A`` and the
  kernel's safe divide (``den > 0`` else 1), ``kernels/parallel_kata.py:193-197``.
* backward clamps ``den`` at ``1e-12`` (``parallel_kata_attn.py:79``).

Every function upcasts its inputs to float64 and returns float64 tensors
(``kata_scores``/``kata_fwd``/``kata_bwd`` take ``work_dtype`` so the bench's
CPU baseline can time the same restatement in float32).
"""

from __future__ import annotations

import math

import torch

F64 = torch.float64


def default_scale(dk: int, num_groups: int) -> float:
    """``1/sqrt(E)`` with ``E = dk // M`` (``parallel_kata_attn.py:152-153``)."""
    return 1.0 / math.sqrt(dk // num_groups)


def _expand_kv(x: torch.Tensor, HQ: int) -> torch.Tensor:
    """Repeat kv heads to the query-head count (``parallel_kata_attn.py:81-95``)."""
    B, T, H, D = x.shape
    G = HQ // H
    if G == 1:
        return x
    return x.unsqueeze(3).expand(B, T, H, G, D).reshape(B, T, HQ, D)


def _group_dots(q, k, M, variant):
    """Raw per-group dot products (no scale).

    concat: ``qk[b,h,t,s,m]`` (``parallel_kata_attn.py:97-100``);
    sum:    ``qk[b,h,t,s,i,j]`` (``parallel_kata_attn.py:613-616``).
    """
    B, T, HQ, dk = q.shape
    E = dk // M
    qg = q.reshape(B, T, HQ, M, E)
    kg = k.reshape(B, T, HQ, M, E)
    if variant == "concat":
        return torch.einsum("bthme,bshme->bhtsm", qg, kg)
    if variant == "sum":
        return torch.einsum("bthie,bshje->bhtsij", qg, kg)
    raise ValueError(f"unknown variant {variant!r}")


def kata_scores(q, k, num_groups, scale=None, variant="concat", c=None, work_dtype=F64):
    """Causal score matrix ``A`` ``(B,HQ,T,T)`` in float64.

    Follows ``kernels/parallel_kata.py:115-191`` (scale applied to the dot
    before squaring; keys after the query masked to zero) and, with a decay
    ``c`` ``(B,T,HQ)``, the extra factor ``exp(min(c_t - c_s, 0))``
    (``kernels/parallel_kata.py:128-133, 169-179``).
    """
    q = q.to(work_dtype)
    k = _expand_kv(k.to(work_dtype), q.shape[2])
    dk = q.shape[-1]
    if scale is None:
        scale = default_scale(dk, num_groups)
    qk = _group_dots(q, k, num_groups, variant) * scale
    if variant == "concat":
        A = (qk * qk).sum(-1)
    else:
        A = (qk * qk).sum(dim=(-2, -1))
    T = q.shape[1]
    causal = torch.tril(torch.ones(T, T, dtype=torch.bool, device=q.device))
    A = A * causal
    if c is not None:
        cH = c.to(work_dtype).transpose(1, 2)  # (B,HQ,T)
        A = A * torch.exp(torch.clamp(cH[..., :, None] - cH[..., None, :], max=0.0))
    return A


def kata_fwd(q, k, v, num_groups=4, scale=None, variant="concat", c=None, work_dtype=F64):
    """Forward ``(o, den)`` in float64: the kernel contract of
    ``parallel_kata_attn_fwd_impl`` (``parallel_kata_attn.py:211-288``) and
    ``parallel_kata_attn_sum_fwd_impl`` (``:539-576``).

    ``o (B,T,HQ,dv)``, ``den (B,T,HQ)``; ``den[t] = sum_{s<=t} A[t,s]``;
    ``o = (A V)/den`` with den replaced by 1 where it is not positive
    (``kernels/parallel_kata.py:193-197``).
    """
    HQ = q.shape[2]
    A = kata_scores(q, k, num_groups, scale, variant, c, work_dtype)  # (B,HQ,T,T)
    vf = _expand_kv(v.to(work_dtype), HQ).permute(0, 2, 1, 3)  # (B,HQ,T,dv)
    num = A @ vf
    den = A.sum(-1)  # (B,HQ,T)
    den_safe = torch.where(den > 0, den, torch.ones_like(den))
    o = num / den_safe[..., None]
    return o.permute(0, 2, 1, 3).contiguous(), den.permute(0, 2, 1).contiguous()


def kata_bwd(q, k, v, o, den, do, num_groups=4, scale=None, variant="concat", work_dtype=F64):
    """Explicit backward ``(dq, dk, dv)`` in float64.

    Restates ``parallel_kata_attn_bwd`` (``parallel_kata_attn.py:49-146``) for
    the concat score and ``parallel_kata_attn_bwd_sum_torch`` (``:579-653``)
    for the sum score: ``P = A/D``, ``delta = <o, dO>``, ``dV = P^T dO``,
    ``dA = (dO V^T - delta)/D`` (causal), ``da = 2 qk dA``,
    ``dQ = scale * da K``, ``dK = scale * da^T Q``; GQA gradients of k and v
    are summed over the query heads sharing a kv head.
    """
    B, T, HQ, dk = q.shape
    H = k.shape[2]
    dv_ = v.shape[-1]
    M = num_groups
    E = dk // M
    G = HQ // H
    if scale is None:
        scale = default_scale(dk, M)
    qf = q.to(work_dtype)
    kf = _expand_kv(k.to(work_dtype), HQ)
    vf = _expand_kv(v.to(work_dtype), HQ)
    dof = do.to(work_dtype)
    Df = den.to(work_dtype).clamp_min(1e-12)
    qk = _group_dots(qf, kf, M, variant) * scale
    if variant == "concat":
        A = (qk * qk).sum(-1)
    else:
        A = (qk * qk).sum(dim=(-2, -1))
    causal = torch.tril(torch.ones(T, T, dtype=torch.bool, device=q.device))
    A = A * causal
    Dh = Df.permute(0, 2, 1)  # (B,HQ,T)
    P = A / Dh[..., None]
    delta = (o.to(work_dtype) * dof).sum(-1).permute(0, 2, 1)  # (B,HQ,T)
    do_p = dof.permute(0, 2, 1, 3)
    v_p = vf.permute(0, 2, 1, 3)
    dV = P.transpose(-1, -2) @ do_p  # (B,HQ,T,dv)
    dA = (do_p @ v_p.transpose(-1, -2) - delta[..., None]) / Dh[..., None]
    dA = dA * causal
    qg = qf.reshape(B, T, HQ, M, E)
    kg = kf.reshape(B, T, HQ, M, E)
    if variant == "concat":
        da = 2.0 * qk * dA[..., None]
        dQ = scale * torch.einsum("bhtsm,bshme->bthme", da, kg)
        dK = scale * torch.einsum("bhtsm,bthme->bshme", da, qg)
    else:
        da = 2.0 * qk * dA[..., None, None]
        dQ = scale * torch.einsum("bhtsij,bshje->bthie", da, kg)
        dK = scale * torch.einsum("bhtsij,bthie->bshje", da, qg)
    dQ = dQ.reshape(B, T, HQ, dk)
    dK = dK.reshape(B, T, HQ, dk)
    dV = dV.permute(0, 2, 1, 3)
    if G > 1:
        dK = dK.reshape(B, T, H, G, dk).sum(3)
        dV = dV.reshape(B, T, H, G, dv_).sum(3)
    return dQ.contiguous(), dK.contiguous(), dV.contiguous()


def kata_decay_ref(q, k, v, c, num_groups, scale):
    """Differentiable decayed KATA forward, restating ``_kata_decay_ref``
    (``parallel_kata_attn.py:291-310``): score times ``exp(min(c_t-c_s,0))``,
    causal, normalised by ``sum + 1e-20``.  Works in the dtype it is given
    (the oracle passes float64 leaves to obtain gradients by autograd, the
    way ``_KataDecayFunction.backward`` does at ``:329-347``).
    """
    B, T, H, Kd = q.shape
    M = num_groups
    E = Kd // M
    qg = q.reshape(B, T, H, M, E)
    kg = k.reshape(B, T, H, M, E)
    qk = torch.einsum("bthme,bshme->bhtsm", qg, kg)
    A = ((scale * qk) ** 2).sum(-1)
    cH = c.transpose(1, 2)
    dec = torch.exp(torch.clamp(cH[:, :, :, None] - cH[:, :, None, :], max=0.0))
    tri = torch.tril(torch.ones(T, T, dtype=A.dtype, device=A.device))
    A = A * dec * tri
    return torch.einsum("bhts,bshd->bthd", A, v) / (
        A.sum(-1).transpose(1, 2)[..., None] + 1e-20
    )


def kata_decay_fwd_bwd(q, k, v, c, do, num_groups, scale=None):
    """``(o, dq, dk, dv, dc)`` of the decayed form via float64 autograd through
    :func:`kata_decay_ref` (the reference's own backward strategy,
    ``parallel_kata_attn.py:329-347``)."""
    if scale is None:
        scale = default_scale(q.shape[-1], num_groups)
    leaves = [x.detach().to(F64).requires_grad_(True) for x in (q, k, v, c)]
    with torch.enable_grad():
        o = kata_decay_ref(*leaves, num_groups, scale)
        grads = torch.autograd.grad(o, leaves, do.to(F64))
    return (o.detach(),) + tuple(g.detach() for g in grads)


# ---------------------------------------------------------------------------
# psi feature maps (kata/references/feature_maps.py)
# ---------------------------------------------------------------------------


def spd_concat(x: torch.Tensor, k_splits: int) -> torch.Tensor:
    """Packed concat-SPD map: per group the diagonal ``g*g`` then the strict
    lower triangle of ``g g^T`` times sqrt(2) (``feature_maps.py:29-58``), so
    ``<psi(x), psi(y)> = sum_g (x_g . y_g)**2``."""
    *prefix, d = x.shape
    if d % k_splits:
        raise ValueError(f"x last dim {d} not divisible by num_splits {k_splits}")
    e = d // k_splits
    g = x.reshape(*prefix, k_splits, e)
    diag = g * g
    if e == 1:
        return diag.reshape(*prefix, k_splits)
    outer = g.unsqueeze(-1) * g.unsqueeze(-2)
    ii, jj = torch.tril_indices(e, e, offset=-1, device=x.device)
    off = outer[..., ii, jj] * math.sqrt(2.0)
    return torch.cat([diag, off], dim=-1).reshape(*prefix, k_splits * (e * (e + 1) // 2))


def spd_full(x: torch.Tensor, num_splits: int) -> torch.Tensor:
    """Full per-group outer product ``vec(g g^T)`` (``feature_maps.py:61-79``)."""
    *prefix, d = x.shape
    e = d // num_splits
    g = x.reshape(*prefix, num_splits, e)
    return (g.unsqueeze(-1) * g.unsqueeze(-2)).reshape(*prefix, num_splits * e * e)


def spd_sum(x: torch.Tensor, num_splits: int) -> torch.Tensor:
    """``vec(sum_i g_i g_i^T)`` (``feature_maps.py:82-98``):
    ``<psi(x), psi(y)> = sum_{i,j} (x_i . y_j)**2``."""
    *prefix, d = x.shape
    e = d // num_splits
    g = x.reshape(*prefix, num_splits, e)
    return torch.einsum("...mi,...mj->...ij", g, g).reshape(*prefix, e * e)


def kata_psi_fwd(q, k, v, num_groups=4, scale=None, variant="concat"):
    """Forward ``(o, den)`` through explicit feature maps: causal linear
    attention with ``psi(sqrt(scale) x)`` (the feature form the reference's
    comments state at ``parallel_kata_attn.py:1-12``).  Independent of
    :func:`kata_fwd`'s dense score computation; the two are checked against
    each other.
    """
    q = q.to(F64)
    k = _expand_kv(k.to(F64), q.shape[2])
    v = _expand_kv(v.to(F64), q.shape[2])
    if scale is None:
        scale = default_scale(q.shape[-1], num_groups)
    s = math.sqrt(scale)
    fmap = spd_concat if variant == "concat" else spd_sum
    pq = fmap(q * s, num_groups)  # (B,T,HQ,P)
    pk = fmap(k * s, num_groups)
    S = torch.cumsum(pk.unsqueeze(-1) * v.unsqueeze(-2), dim=1)  # (B,T,HQ,P,dv)
    z = torch.cumsum(pk, dim=1)  # (B,T,HQ,P)
    num = torch.einsum("bthp,bthpv->bthv", pq, S)
    den = (pq * z).sum(-1)
    den_safe = torch.where(den > 0, den, torch.ones_like(den))
    return num / den_safe[..., None], den


# ---------------------------------------------------------------------------
# O(T) state form: long-context prefill and recurrent decode
# ---------------------------------------------------------------------------


def kata_state_prefill(k, v, num_groups=4, scale=None):
    """Concat psi-state after a prefill, float64, in the full (unpacked)
    per-group form of ``spd_chunk_scan_cat`` (``kata/spd/chunk_scan_cat.py:219-345``):
    ``S[b,h] = sum_s psi(s k_s) v_s^T`` ``(B,H,M*E*E,dv)`` and
    ``z[b,h] = sum_s psi(s k_s)`` ``(B,H,M*E*E)`` with ``s = sqrt(scale)``.
    Inputs time-major ``(B,T,H,D)``.
    """
    k = k.to(F64)
    v = v.to(F64)
    if scale is None:
        scale = default_scale(k.shape[-1], num_groups)
    s = math.sqrt(scale)
    pk = spd_full(k * s, num_groups)  # (B,T,H,P)
    S = torch.einsum("bthp,bthv->bhpv", pk, v)
    z = pk.sum(1)
    return S, z


def kata_decode_step(S, z, q, k, v, num_groups=4, scale=None, eps=1e-6):
    """One recurrent decode step on the concat psi-state (float64).

    ``S (B,H,M*E*E,dv)``, ``z (B,H,M*E*E)``, ``q,k,v (B,H,D)``.  The state is
    updated with the new key first (causal, ``s <= t``), then read out as
    ``o = psi(s q)^T S / max(psi(s q).z, eps)`` - the ``EPS`` floor of the
    reference's state readout (``kata/spd/chunk_scan_cat.py:188-191``).
    The reference's flash path keeps no decode state (``kata/layer.py:492``);
    this form is pinned by equality with row ``n`` of the parallel form.
    Returns ``(o (B,H,dv), S', z')``.
    """
    if scale is None:
        scale = default_scale(q.shape[-1], num_groups)
    s = math.sqrt(scale)
    q, k, v = (x.to(F64) for x in (q, k, v))
    pk = spd_full(k * s, num_groups)
    pq = spd_full(q * s, num_groups)
    S = S + pk.unsqueeze(-1) * v.unsqueeze(-2)
    z = z + pk
    num = torch.einsum("bhp,bhpv->bhv", pq, S)
    den = torch.clamp((pq * z).sum(-1), min=eps)
    return num / den[..., None], S, z


def psi_features(x, num_groups, feature="quad"):
    """The tree-scan's feature map (``kata/spd/chunk_scan_cat.py:90-98``):
    ``"quad"`` is psi(x) = vec(x_g x_g^T) per group, ``"linear"`` psi(x) = x_g,
    which concatenated over the groups is x itself."""
    return spd_full(x, num_groups) if feature == "quad" else x


def kata_prefill_fwd_state_form(q, k, v, num_groups=4, scale=None, chunk=64, eps=1e-6,
                                feature="quad"):
    """Chunked O(T) prefill output ``(o, den)`` in the state form (float64):
    per chunk, inter-chunk ``psi(sq) S_prev`` plus the intra-chunk causal
    block, normalised with the EPS floor of ``chunk_scan_cat.py:188-191``.
    Returns also the final ``(S, z)``.  ``feature`` as ``psi_features``.
    """
    B, T, H, D = q.shape
    if scale is None:
        scale = default_scale(D, num_groups)
    s = math.sqrt(scale)
    q, k, v = (x.to(F64) for x in (q, k, v))
    P = num_groups * (D // num_groups) ** 2 if feature == "quad" else D
    S = torch.zeros(B, H, P, v.shape[-1], dtype=F64, device=q.device)
    z = torch.zeros(B, H, P, dtype=F64, device=q.device)
    outs, dens = [], []
    for c0 in range(0, T, chunk):
        qc, kc, vc = q[:, c0:c0 + chunk], k[:, c0:c0 + chunk], v[:, c0:c0 + chunk]
        pq = psi_features(qc * s, num_groups, feature)  # (B,C,H,P)
        pk = psi_features(kc * s, num_groups, feature)
        Cn = qc.shape[1]
        A = torch.einsum("bthp,bshp->bhts", pq, pk) * torch.tril(
            torch.ones(Cn, Cn, dtype=F64, device=q.device))
        num = torch.einsum("bthp,bhpv->bthv", pq, S) + torch.einsum("bhts,bshv->bthv", A, vc)
        den = torch.einsum("bthp,bhp->bth", pq, z) + A.sum(-1).transpose(1, 2)
        den = torch.clamp(den, min=eps)
        outs.append(num / den[..., None])
        dens.append(den)
        S = S + torch.einsum("bshp,bshv->bhpv", pk, vc)
        z = z + pk.sum(1)
    return torch.cat(outs, 1), torch.cat(dens, 1), S, z


def linear_attn_dense(q, k, v, scale, eps=1e-6):
    """Dense causal form of the tree-scan's linear feature (float64,
    time-major ``(B, T, H, D)``): kappa = scale q.k, den_t = max(sum_{s<=t}
    kappa, eps) (``kata/spd/chunk_scan_cat.py:188-191``), o = num / den."""
    q, k, v = (x.to(F64) for x in (q, k, v))
    T = q.shape[1]
    A = scale * torch.einsum("bthd,bshd->bhts", q, k) * torch.tril(torch.ones(T, T, dtype=F64))
    num = torch.einsum("bhts,bshv->bthv", A, v)
    den = torch.clamp(A.sum(-1).transpose(1, 2), min=eps)
    return num / den[..., None], den
