"""Float64 CPU restatement of the reference's SPD delta rule (DeltaKata,
``flash_delta``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference: ``kata/spd/flash_delta.py`` -- the pseudo-value solve
``_flash_U_kernel`` (``:25-183``), the readout ``_readout_kernel``
(``:898-972``), the denominator ``_den_kernel`` (``:986-1046``) and the
autograd op ``_FlashDelta`` / ``flash_delta`` (``:1060-1116``), reached from
the mixer's delta branch (``kata/layer.py:377-420``) for
``configs/model/kata_delta_m1_340m.yaml:22``.

Conventions (time-major ``(B, T, H, D)``; ``M`` groups of ``E = D / M``):

* ``s = sqrt(scale)``, ``scale=None`` means ``1/E`` (``flash_delta.py:191-193,
  837``), applied to both q and k;
* the sum-SPD kernel ``kappa(a, b) = sum_{g,h} (s a_g . s b_h)^2``
  (``:67-103, 240-266``);
* ``A_kk[t, u] = kappa(k_t, k_u)``, ``A_qk[t, u] = kappa(q_t, k_u)``;
* pseudo-values ``U = (I + diag(beta) tril(A_kk, -1))^{-1} diag(beta) V``
  (``:1-10, 134-183``);
* ``num = tril(A_qk) U`` (diagonal included, ``:958-961``);
  ``den_t = sum_{u <= t} A_qk[t, u]`` (``:1040-1042``);
* ``o = num / (den + eps)`` when ``normalize`` else ``o = num`` (``:1063-1069``).

This is the delta rule with queries and keys lifted to the feature
``phi(x) = s^2 vec(sum_g x_g x_g^T)`` (``<phi(a), phi(b)> = kappa(a, b)``):
``S_t = S_{t-1} + beta_t phi(k_t) (v_t - S_{t-1}^T phi(k_t))^T``,
``num_t = S_t^T phi(q_t)``.  :func:`flash_delta_recurrent` computes that
recurrence; the tests check the dense form against it.
"""

from __future__ import annotations

import torch

F64 = torch.float64


def _scale(D, M, scale):
    return 1.0 / (D // M) if scale is None else float(scale)


def kappa_gram(a, b, M, scale=None):
    """``G[bb, h, t, u] = sum_{g,h'} (s a[bb,t,h,g] . s b[bb,u,h,h'])^2``
    (``flash_delta.py:240-266``), float64."""
    B, T, H, D = a.shape
    E = D // M
    s2 = _scale(D, M, scale)
    ag = a.to(F64).reshape(B, T, H, M, E)
    bg = b.to(F64).reshape(B, b.shape[1], H, M, E)
    dots = torch.einsum("bthge,buhke->bhtugk", ag, bg) * s2
    return (dots * dots).sum((-2, -1))


def flash_delta_U(k, v, beta, M, scale=None):
    """Pseudo-values ``U (B, T, H, DV)`` by a dense triangular solve
    (``flash_delta.py:25-183``)."""
    B, T, H, _ = k.shape
    A = kappa_gram(k, k, M, scale)                       # (B, H, T, T)
    bt = beta.to(F64).permute(0, 2, 1)                   # (B, H, T)
    L = torch.eye(T, dtype=F64) + bt[..., :, None] * torch.tril(A, -1)
    rhs = bt[..., None] * v.to(F64).permute(0, 2, 1, 3)  # (B, H, T, DV)
    U = torch.linalg.solve_triangular(L, rhs, upper=False, unitriangular=True)
    return U.permute(0, 2, 1, 3).contiguous()


def flash_delta_fwd(q, k, v, beta, M, scale=None, normalize=False, eps=1e-5):
    """``(o, U, num, den)`` of ``flash_delta`` in float64
    (``flash_delta.py:1060-1116``)."""
    U = flash_delta_U(k, v, beta, M, scale)
    Aqk = torch.tril(kappa_gram(q, k, M, scale))         # (B, H, T, T)
    num = torch.einsum("bhtu,buhd->bthd", Aqk, U)
    den = Aqk.sum(-1).permute(0, 2, 1).contiguous()      # (B, T, H)
    o = num / (den[..., None] + eps) if normalize else num
    return o, U, num, den


def flash_delta_recurrent(q, k, v, beta, M, scale=None):
    """Per-token delta rule on the explicit feature ``phi(x) = s^2 vec(sum_g
    x_g x_g^T)`` (E^2 features): returns ``num (B, T, H, DV)`` and the final
    state ``S (B, H, E^2, DV)``.  Independent of the dense Gram / solve form."""
    B, T, H, D = q.shape
    E = D // M
    s2 = _scale(D, M, scale)

    def phi(x):
        g = x.to(F64).reshape(*x.shape[:-1], M, E)
        return s2 * torch.einsum("...gi,...gj->...ij", g, g).reshape(*x.shape[:-1], E * E)

    pq, pk = phi(q), phi(k)
    S = torch.zeros(B, H, E * E, v.shape[-1], dtype=F64)
    outs = []
    for t in range(T):
        kt, vt, bt = pk[:, t], v[:, t].to(F64), beta[:, t].to(F64)
        u = bt[..., None] * (vt - torch.einsum("bhp,bhpd->bhd", kt, S))
        S = S + kt[..., :, None] * u[..., None, :]
        outs.append(torch.einsum("bhp,bhpd->bhd", pq[:, t], S))
    return torch.stack(outs, 1), S


def flash_delta_fwd_bwd(q, k, v, beta, M, do, scale=None, normalize=False, eps=1e-5):
    """float64 ``o`` and the gradients ``dq, dk, dv, dbeta`` of ``<o, do>``
    by autograd through :func:`flash_delta_fwd` (the reference's
    ``_FlashDelta.backward``, ``flash_delta.py:1084-1108``, differentiates
    the same function)."""
    leaves = [t.detach().to(F64).requires_grad_(True) for t in (q, k, v, beta)]
    with torch.enable_grad():
        o = flash_delta_fwd(*leaves, M, scale, normalize, eps)[0]
        grads = torch.autograd.grad((o * do.to(F64)).sum(), leaves)
    return (o.detach(), *[g.detach() for g in grads])
