"""Float64 CPU restatement of the (gated) delta rule.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference reaches this arithmetic only through the third-party package
``flash-linear-attention==0.5.0`` (``fla``; pinned at ``scripts/setup.sh:27``
and ``README.md:44``), via ``model_type: delta_net`` /
``gated_deltanet`` (``configs/model/200m/delta_net_200m.yaml:3``,
``configs/model/200m/gated_deltanet_200m.yaml:4``).  ``fla`` is absent from
this container, so the algorithm is restated from its published form:

* DeltaNet (Schlag et al. 2021; chunked WY form: Yang, Wang, Zhang, Shen,
  Kim, "Parallelizing Linear Transformers with the Delta Rule over Sequence
  Length", NeurIPS 2024):
  ``S_t = S_{t-1} + beta_t k_t (v_t - S_{t-1}^T k_t)^T``, ``o_t = scale S_t^T q_t``.
* GatedDeltaNet (Yang, Kautz, Hatamizadeh, ICLR 2025):
  ``S_t = a_t S_{t-1} + beta_t k_t (v_t - a_t S_{t-1}^T k_t)^T`` with
  ``a_t = exp(g_t)``.

Layout follows fla's public API: q, k ``(B,T,H,K)``, v ``(B,T,H,V)``,
beta and g ``(B,T,H)``, states ``(B,H,K,V)``; ``scale=None`` means
``1/sqrt(K)``.  Parity with fla itself is unpinned (no fla outputs exist in
the reference); the naive recurrence is the ground truth and the chunked
form must match it.
"""

from __future__ import annotations

import math

import torch

F64 = torch.float64


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Row L2 normalisation ``x / sqrt(sum x^2 + eps)`` (the form of fla's
    ``l2norm`` used by ``use_qk_l2norm_in_kernel``)."""
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


def delta_rule_recurrent(q, k, v, beta, g=None, scale=None, initial_state=None,
                         use_qk_l2norm=False):
    """Naive per-token recurrence (ground truth). Works in the dtype of its
    inputs (the tests pass float64 leaves and differentiate through it).

    Returns ``(o (B,T,H,V), S_T (B,H,K,V))``.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(K)
    if use_qk_l2norm:
        q, k = l2norm(q), l2norm(k)
    S = (initial_state if initial_state is not None
         else torch.zeros(B, H, K, V, dtype=q.dtype, device=q.device))
    outs = []
    for t in range(T):
        qt, kt, vt, bt = q[:, t], k[:, t], v[:, t], beta[:, t]
        if g is not None:
            S = S * torch.exp(g[:, t])[..., None, None]
        u = bt[..., None] * (vt - torch.einsum("bhk,bhkv->bhv", kt, S))
        S = S + kt[..., :, None] * u[..., None, :]
        outs.append(scale * torch.einsum("bhk,bhkv->bhv", qt, S))
    return torch.stack(outs, 1), S


def delta_rule_chunked(q, k, v, beta, g=None, scale=None, initial_state=None,
                       chunk=64, use_qk_l2norm=False):
    """Chunked WY/UT form (float64 or the dtype given; differentiable).

    Per chunk with ``G = cumsum_chunk(g)`` (zero when ungated):

    1. ``A = tril(diag(beta) K K^T * exp(G_i - G_j), -1)``
    2. ``Tm = (I + A)^{-1}``
    3. ``W = Tm diag(beta * exp(G)) K``,  ``U = Tm diag(beta) V``
    4. ``v_new = U - W S_c``
    5. ``o = scale (diag(exp(G)) Q S_c + tril(Q K^T * exp(G_i - G_j)) v_new)``
    6. ``S_{c+1} = exp(G_C) S_c + (K * exp(G_C - G))^T v_new``

    Returns ``(o, S_T)``.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(K)
    if use_qk_l2norm:
        q, k = l2norm(q), l2norm(k)
    dt = q.dtype
    dev = q.device
    S = (initial_state if initial_state is not None
         else torch.zeros(B, H, K, V, dtype=dt, device=dev))
    qh, kh, vh = (x.transpose(1, 2) for x in (q, k, v))  # (B,H,T,D)
    bh = beta.transpose(1, 2)  # (B,H,T)
    gh = g.transpose(1, 2) if g is not None else None
    outs = []
    for c0 in range(0, T, chunk):
        Qc, Kc, Vc = qh[:, :, c0:c0 + chunk], kh[:, :, c0:c0 + chunk], vh[:, :, c0:c0 + chunk]
        bc = bh[:, :, c0:c0 + chunk]
        C = Qc.shape[2]
        if gh is not None:
            Gc = torch.cumsum(gh[:, :, c0:c0 + chunk], -1)
        else:
            Gc = torch.zeros(B, H, C, dtype=dt, device=dev)
        Dg = torch.exp(Gc[..., :, None] - Gc[..., None, :])  # (B,H,C,C)
        strict = torch.tril(torch.ones(C, C, dtype=torch.bool, device=dev), -1)
        lower = torch.tril(torch.ones(C, C, dtype=torch.bool, device=dev))
        A = (bc[..., :, None] * (Kc @ Kc.transpose(-1, -2)) * Dg).masked_fill(~strict, 0.0)
        eye = torch.eye(C, dtype=dt, device=dev).expand(B, H, C, C)
        Tm = torch.linalg.solve_triangular(eye + A, eye, upper=False, unitriangular=True)
        W = Tm @ (Kc * (bc * torch.exp(Gc))[..., None])
        U = Tm @ (Vc * bc[..., None])
        vnew = U - W @ S
        Aqk = ((Qc @ Kc.transpose(-1, -2)) * Dg).masked_fill(~lower, 0.0)
        o = scale * ((Qc * torch.exp(Gc)[..., None]) @ S + Aqk @ vnew)
        outs.append(o)
        gl = Gc[..., -1]
        S = (S * torch.exp(gl)[..., None, None]
             + (Kc * torch.exp(gl[..., None] - Gc)[..., None]).transpose(-1, -2) @ vnew)
    o = torch.cat(outs, 2).transpose(1, 2).contiguous()
    return o, S


def delta_rule_fwd_bwd(q, k, v, beta, g=None, scale=None, initial_state=None,
                       do=None, dht=None, chunk=64, use_qk_l2norm=False,
                       form="chunked"):
    """Float64 forward and autograd backward.

    Returns a dict with ``o, ht`` and the gradients ``dq, dk, dv, dbeta``
    (plus ``dg`` when gated and ``dh0`` when an initial state is given)
    for the loss ``<o, do> + <ht, dht>``.
    """
    names = ["q", "k", "v", "beta"]
    tens = [q, k, v, beta]
    if g is not None:
        names.append("g")
        tens.append(g)
    if initial_state is not None:
        names.append("h0")
        tens.append(initial_state)
    leaves = [t.detach().to(F64).requires_grad_(True) for t in tens]
    d = dict(zip(names, leaves))
    fn = delta_rule_chunked if form == "chunked" else delta_rule_recurrent
    kw = dict(g=d.get("g"), scale=scale, initial_state=d.get("h0"),
              use_qk_l2norm=use_qk_l2norm)
    if form == "chunked":
        kw["chunk"] = chunk
    with torch.enable_grad():
        o, ht = fn(d["q"], d["k"], d["v"], d["beta"], **kw)
        loss = (o * do.to(F64)).sum() if do is not None else o.sum() * 0
        if dht is not None:
            loss = loss + (ht * dht.to(F64)).sum()
        grads = torch.autograd.grad(loss, leaves)
    out = {"o": o.detach(), "ht": ht.detach()}
    for n, gr in zip(names, grads):
        out["d" + n] = gr.detach()
    return out
