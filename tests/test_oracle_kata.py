"""Pins the KATA oracle (``oracle/kata.py``) without trusting its own formulas.

Each check is chosen so that a plausible mistake in the oracle (a dropped
group, scale applied after squaring, a transposed operand, a wrong causal
edge, a missing GQA reduction, a sign slip in the backward) fails at least one:

* brute force: pure-Python loops over (t, s, g, e) at T <= 6;
* two independent forward forms: dense scores vs. psi-feature prefix sums
  (``spd_concat`` / ``spd_sum`` of ``kata/references/feature_maps.py``);
* invariants: constant v gives constant o, o_0 = v_0, M=1 concat == M=1 sum,
  consistent group permutation leaves A unchanged, A >= 0;
* backward: the explicit formulas vs. float64 autograd through the dense form,
  and finite differences (``torch.autograd.gradcheck``);
* decay: c == 0 reduces to concat; for c_t = -lam t the output equals an
  independent decayed psi-state recurrence (S <- e^{-lam} S + psi(k) v^T);
  c -> c + const changes nothing; a pure-Python brute force with a
  non-monotone c pins the clamp min(c_t - c_s, 0), its sign and its scale;
* state form: prefill state equals the psi sums, decode after n tokens equals
  row n of the parallel form, chunked state-form prefill equals the dense form.
"""

import math

import pytest
import torch

from oracle import kata as K

F64 = torch.float64


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=F64) * scale


def _brute_fwd(q, k, v, M, scale, variant):
    B, T, HQ, dk = q.shape
    H = k.shape[2]
    G = HQ // H
    E = dk // M
    dv = v.shape[-1]
    o = torch.zeros(B, T, HQ, dv, dtype=F64)
    den = torch.zeros(B, T, HQ, dtype=F64)
    for b in range(B):
        for hq in range(HQ):
            h = hq // G
            for t in range(T):
                acc = [0.0] * dv
                d = 0.0
                for s in range(t + 1):
                    a = 0.0
                    if variant == "concat":
                        for gi in range(M):
                            dot = sum(float(q[b, t, hq, gi * E + e]) * float(k[b, s, h, gi * E + e])
                                      for e in range(E))
                            a += (scale * dot) ** 2
                    else:
                        for gi in range(M):
                            for gj in range(M):
                                dot = sum(float(q[b, t, hq, gi * E + e]) * float(k[b, s, h, gj * E + e])
                                          for e in range(E))
                                a += (scale * dot) ** 2
                    d += a
                    for j in range(dv):
                        acc[j] += a * float(v[b, s, h, j])
                den[b, t, hq] = d
                for j in range(dv):
                    o[b, t, hq, j] = acc[j] / (d if d > 0 else 1.0)
    return o, den


@pytest.mark.parametrize("variant", ["concat", "sum"])
@pytest.mark.parametrize("M", [1, 2, 4])
def test_fwd_brute_force(variant, M):
    B, T, H, dk, dv = 1, 5, 2, 8, 3
    q, k, v = _rand((B, T, H, dk), 1), _rand((B, T, H, dk), 2), _rand((B, T, H, dv), 3)
    scale = 0.7
    o, den = K.kata_fwd(q, k, v, M, scale, variant)
    ob, denb = _brute_fwd(q, k, v, M, scale, variant)
    torch.testing.assert_close(o, ob, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(den, denb, rtol=1e-12, atol=1e-12)


def test_fwd_brute_force_gqa():
    B, T, HQ, H, dk, dv = 2, 4, 4, 2, 8, 2
    q, k, v = _rand((B, T, HQ, dk), 4), _rand((B, T, H, dk), 5), _rand((B, T, H, dv), 6)
    o, den = K.kata_fwd(q, k, v, 2, None, "concat")
    ob, denb = _brute_fwd(q, k, v, 2, 1 / math.sqrt(4), "concat")
    torch.testing.assert_close(o, ob, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(den, denb, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("variant", ["concat", "sum"])
@pytest.mark.parametrize("M", [1, 2, 4])
def test_dense_vs_psi_form(variant, M):
    B, T, H, dk, dv = 2, 37, 3, 16, 8
    q, k, v = _rand((B, T, H, dk), 7), _rand((B, T, H, dk), 8), _rand((B, T, H, dv), 9)
    o1, d1 = K.kata_fwd(q, k, v, M, None, variant)
    o2, d2 = K.kata_psi_fwd(q, k, v, M, None, variant)
    torch.testing.assert_close(o1, o2, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(d1, d2, rtol=1e-10, atol=1e-10)


def test_invariants():
    B, T, H, dk, dv = 2, 19, 2, 16, 4
    q, k = _rand((B, T, H, dk), 10), _rand((B, T, H, dk), 11)
    v = _rand((B, T, H, dv), 12)
    # constant v -> constant o (rows are convex combinations)
    vc = torch.ones(B, T, H, dv, dtype=F64) * 3.25
    o, _ = K.kata_fwd(q, k, vc, 4)
    torch.testing.assert_close(o, vc, rtol=1e-12, atol=1e-12)
    # first row attends only to itself
    o, den = K.kata_fwd(q, k, v, 4)
    torch.testing.assert_close(o[:, 0], v[:, 0], rtol=1e-12, atol=1e-12)
    # scores are non-negative
    assert (K.kata_scores(q, k, 4) >= 0).all()
    # M=1 concat == M=1 sum
    oc, dc = K.kata_fwd(q, k, v, 1, None, "concat")
    os_, ds = K.kata_fwd(q, k, v, 1, None, "sum")
    torch.testing.assert_close(oc, os_)
    torch.testing.assert_close(dc, ds)
    # permuting the groups of q and k together leaves concat scores unchanged
    perm = torch.tensor([2, 0, 3, 1])
    qp = q.reshape(B, T, H, 4, 4)[..., perm, :].reshape(B, T, H, dk)
    kp = k.reshape(B, T, H, 4, 4)[..., perm, :].reshape(B, T, H, dk)
    torch.testing.assert_close(K.kata_scores(q, k, 4), K.kata_scores(qp, kp, 4))
    # ... and permuting only k's groups changes them (the pairing matters)
    assert not torch.allclose(K.kata_scores(q, k, 4), K.kata_scores(q, kp, 4))
    # normalised output does not depend on scale; den scales with scale**2
    o2, den2 = K.kata_fwd(q, k, v, 4, scale=0.5)
    o3, den3 = K.kata_fwd(q, k, v, 4, scale=1.5)
    torch.testing.assert_close(o2, o3)
    torch.testing.assert_close(den3, den2 * 9.0)


def _dense_autograd(q, k, v, do, M, scale, variant):
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v)]
    o, _ = K.kata_fwd(*leaves, M, scale, variant)
    return torch.autograd.grad((o * do).sum(), leaves)


@pytest.mark.parametrize("variant", ["concat", "sum"])
@pytest.mark.parametrize("M,HQ,H", [(1, 2, 2), (2, 2, 2), (4, 3, 3), (2, 4, 2)])
def test_bwd_explicit_vs_autograd(variant, M, HQ, H):
    B, T, dk, dv = 2, 23, 16, 8
    q, k, v = _rand((B, T, HQ, dk), 13), _rand((B, T, H, dk), 14), _rand((B, T, H, dv), 15)
    do = _rand((B, T, HQ, dv), 16)
    o, den = K.kata_fwd(q, k, v, M, None, variant)
    dq, dk_, dv_ = K.kata_bwd(q, k, v, o, den, do, M, None, variant)
    gq, gk, gv = _dense_autograd(q, k, v, do, M, None, variant)
    torch.testing.assert_close(dq, gq, rtol=1e-9, atol=1e-10)
    torch.testing.assert_close(dk_, gk, rtol=1e-9, atol=1e-10)
    torch.testing.assert_close(dv_, gv, rtol=1e-9, atol=1e-10)


def test_bwd_finite_differences():
    B, T, H, dk, dv = 1, 6, 1, 4, 3
    q, k, v = (_rand((B, T, H, dk), 17).requires_grad_(True),
               _rand((B, T, H, dk), 18).requires_grad_(True),
               _rand((B, T, H, dv), 19).requires_grad_(True))
    assert torch.autograd.gradcheck(lambda a, b, c: K.kata_fwd(a, b, c, 2)[0], (q, k, v))


def test_decay_reduces_and_matches_ref():
    B, T, H, dk, dv = 2, 21, 2, 16, 8
    q, k, v = _rand((B, T, H, dk), 20), _rand((B, T, H, dk), 21), _rand((B, T, H, dv), 22)
    zero = torch.zeros(B, T, H, dtype=F64)
    o0, _ = K.kata_fwd(q, k, v, 2, None, "concat", c=zero)
    o1, _ = K.kata_fwd(q, k, v, 2)
    torch.testing.assert_close(o0, o1)
    c = -torch.cumsum(torch.rand(B, T, H, generator=torch.Generator().manual_seed(3), dtype=F64), 1)
    od, _ = K.kata_fwd(q, k, v, 2, None, "concat", c=c)
    orf = K.kata_decay_ref(q, k, v, c, 2, K.default_scale(dk, 2))
    torch.testing.assert_close(od, orf, rtol=1e-10, atol=1e-12)
    # decay strictly changes the result when c is not constant
    assert not torch.allclose(od, o1)
    # dc gradient by finite differences
    cc = c.clone().requires_grad_(True)
    assert torch.autograd.gradcheck(
        lambda x: K.kata_decay_ref(q[:, :6], k[:, :6], v[:, :6], x, 2, 0.5), (cc[:, :6].detach().requires_grad_(True),))


def test_state_form():
    B, T, H, D, dv, M = 1, 40, 2, 8, 4, 2
    q, k, v = _rand((B, T, H, D), 23), _rand((B, T, H, D), 24), _rand((B, T, H, dv), 25)
    # prefill state equals sums of explicit outer products
    S, z = K.kata_state_prefill(k, v, M)
    E = D // M
    s = math.sqrt(1 / math.sqrt(E))
    for b in range(B):
        for h in range(H):
            Sb = torch.zeros(M * E * E, dv, dtype=F64)
            zb = torch.zeros(M * E * E, dtype=F64)
            for t in range(T):
                for g in range(M):
                    kg = k[b, t, h, g * E:(g + 1) * E] * s
                    blk = torch.outer(kg, kg).reshape(-1)
                    Sb[g * E * E:(g + 1) * E * E] += blk[:, None] * v[b, t, h][None, :]
                    zb[g * E * E:(g + 1) * E * E] += blk
            torch.testing.assert_close(S[b, h], Sb)
            torch.testing.assert_close(z[b, h], zb)
    # decode after an n-token prefill equals row n of the parallel form
    n = T - 1
    S, z = K.kata_state_prefill(k[:, :n], v[:, :n], M)
    o_dec, S2, z2 = K.kata_decode_step(S, z, q[:, n], k[:, n], v[:, n], M)
    o_par, _ = K.kata_fwd(q, k, v, M)
    torch.testing.assert_close(o_dec, o_par[:, n])
    Sf, zf = K.kata_state_prefill(k, v, M)
    torch.testing.assert_close(S2, Sf)
    torch.testing.assert_close(z2, zf)
    # chunked state-form prefill output equals the dense form
    o_sf, den_sf, S3, z3 = K.kata_prefill_fwd_state_form(q, k, v, M, chunk=16)
    torch.testing.assert_close(o_sf, o_par)
    torch.testing.assert_close(S3, Sf)


def test_feature_map_inner_products():
    x, y = _rand((5, 12), 26), _rand((5, 12), 27)
    for M in (1, 2, 3, 4, 6):
        E = 12 // M
        want = sum((x[:, g * E:(g + 1) * E] * y[:, g * E:(g + 1) * E]).sum(-1) ** 2 for g in range(M))
        torch.testing.assert_close((K.spd_concat(x, M) * K.spd_concat(y, M)).sum(-1), want)
        torch.testing.assert_close((K.spd_full(x, M) * K.spd_full(y, M)).sum(-1), want)
        want_sum = sum((x[:, i * E:(i + 1) * E] * y[:, j * E:(j + 1) * E]).sum(-1) ** 2
                       for i in range(M) for j in range(M))
        torch.testing.assert_close((K.spd_sum(x, M) * K.spd_sum(y, M)).sum(-1), want_sum)


# ---------------------------------------------------------------------------
# Decay factor exp(min(c_t - c_s, 0)) (reference kata/parallel_kata_attn.py:291-310,
# c from kata/layer.py:440-447), pinned without the oracle's own formula.
# ---------------------------------------------------------------------------


def _decayed_psi_recurrence(q, k, v, lam, M, scale):
    """Independent form for c_t = -lam * t: the psi-state recurrence with a
    per-step forgetting factor, S <- e^{-lam} S + psi(k) v^T and
    z <- e^{-lam} z + psi(k), o_t = psi(q_t)^T S / psi(q_t).z, den_t =
    scale^2 psi(q_t).z (psi from feature_maps.py:29-58 via spd_concat)."""
    B, T, H, dk = q.shape
    pq, pk = K.spd_concat(q, M), K.spd_concat(k, M)
    P, dv = pq.shape[-1], v.shape[-1]
    S = torch.zeros(B, H, P, dv, dtype=F64)
    z = torch.zeros(B, H, P, dtype=F64)
    a = math.exp(-lam)
    os_, dens = [], []
    for t in range(T):
        S = a * S + pk[:, t, :, :, None] * v[:, t, :, None, :]
        z = a * z + pk[:, t]
        num = torch.einsum("bhp,bhpd->bhd", pq[:, t], S)
        dn = (pq[:, t] * z).sum(-1)
        os_.append(num / dn[..., None])
        dens.append(scale * scale * dn)
    return torch.stack(os_, 1), torch.stack(dens, 1)


@pytest.mark.parametrize("lam", [0.0, 0.05, 0.7])
def test_decay_linear_c_equals_decayed_recurrence(lam):
    B, T, H, dk, dv, M = 2, 19, 2, 8, 5, 2
    q, k, v = _rand((B, T, H, dk), 40), _rand((B, T, H, dk), 41), _rand((B, T, H, dv), 42)
    t = torch.arange(T, dtype=F64)
    c = (-lam * t)[None, :, None].expand(B, T, H).contiguous()
    scale = K.default_scale(dk, M)
    want_o, want_den = _decayed_psi_recurrence(q, k, v, lam, M, scale)
    o, den = K.kata_fwd(q, k, v, M, None, "concat", c=c)
    torch.testing.assert_close(o, want_o, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(den, want_den, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(K.kata_decay_ref(q, k, v, c, M, scale), want_o, rtol=1e-10, atol=1e-12)


def test_decay_shift_invariance():
    # only differences c_t - c_s enter: c -> c + const leaves o and den unchanged
    B, T, H, dk, dv, M = 1, 17, 3, 8, 4, 4
    q, k, v = _rand((B, T, H, dk), 43), _rand((B, T, H, dk), 44), _rand((B, T, H, dv), 45)
    c = -torch.cumsum(torch.rand(B, T, H, generator=torch.Generator().manual_seed(46), dtype=F64), 1)
    o1, d1 = K.kata_fwd(q, k, v, M, None, "concat", c=c)
    o2, d2 = K.kata_fwd(q, k, v, M, None, "concat", c=c + 3.25)
    torch.testing.assert_close(o1, o2, rtol=1e-12, atol=1e-13)
    torch.testing.assert_close(d1, d2, rtol=1e-12, atol=1e-13)


def _brute_decay(q, k, v, c, M, scale, clamp=True):
    """Pure-Python loops: A[t,s] = sum_g (scale q_g.k_g)^2 * exp(min(c_t - c_s, 0)),
    s <= t; o = sum A v / (sum A + 1e-20) (parallel_kata_attn.py:291-310)."""
    B, T, H, dk = q.shape
    E, dv = dk // M, v.shape[-1]
    o = torch.zeros(B, T, H, dv, dtype=F64)
    for b in range(B):
        for h in range(H):
            for t in range(T):
                num = [0.0] * dv
                den = 0.0
                for s in range(t + 1):
                    a = 0.0
                    for g in range(M):
                        d = sum(float(q[b, t, h, g * E + e]) * float(k[b, s, h, g * E + e]) for e in range(E))
                        a += (scale * d) ** 2
                    dc = float(c[b, t, h]) - float(c[b, s, h])
                    a *= math.exp(min(dc, 0.0) if clamp else dc)
                    den += a
                    for j in range(dv):
                        num[j] += a * float(v[b, s, h, j])
                for j in range(dv):
                    o[b, t, h, j] = num[j] / (den + 1e-20)
    return o


def test_decay_brute_force_non_monotone_c():
    # c is NOT cumulative here: c_t - c_s takes both signs, so the clamp at 0,
    # the sign of the difference and the exponent scale are all exercised
    B, T, H, dk, dv, M = 1, 6, 2, 4, 3, 2
    q, k, v = _rand((B, T, H, dk), 47), _rand((B, T, H, dk), 48), _rand((B, T, H, dv), 49)
    c = _rand((B, T, H), 50, 1.5)
    scale = 0.7
    want = _brute_decay(q, k, v, c, M, scale)
    got, _ = K.kata_fwd(q, k, v, M, scale, "concat", c=c)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-13)
    torch.testing.assert_close(K.kata_decay_ref(q, k, v, c, M, scale), want, rtol=1e-12, atol=1e-13)
    # plausible mistakes are visible at this size: no clamp, or no decay at all
    assert (_brute_decay(q, k, v, c, M, scale, clamp=False) - want).abs().max() > 1e-3
    assert (K.kata_fwd(q, k, v, M, scale, "concat")[0] - want).abs().max() > 1e-3


def test_linear_feature():
    """The tree-scan's linear feature (``kata/spd/chunk_scan_cat.py:90-92``):
    the chunked state form equals the dense causal form and a token-by-token
    loop, the group split drops out, and den is clamped at eps (where it is
    negative, o = num / eps)."""
    B, T, H, D, dv = 1, 50, 2, 8, 4
    q, k, v = _rand((B, T, H, D), 41), _rand((B, T, H, D), 42), _rand((B, T, H, dv), 43)
    scale, eps = 0.3, 1e-6
    o_d, den_d = K.linear_attn_dense(q, k, v, scale, eps)
    assert (den_d == eps).any() and (den_d > eps).any()  # both sides of the clamp occur
    for M, C in ((1, 64), (2, 7), (4, 16)):
        o_s, den_s, S, z = K.kata_prefill_fwd_state_form(q, k, v, M, scale, C, eps, feature="linear")
        torch.testing.assert_close(o_s, o_d)
        torch.testing.assert_close(den_s, den_d)
        assert S.shape == (B, H, D, dv) and z.shape == (B, H, D)
    # token-by-token: S_t = S_{t-1} + k_t v_t^T, z_t = z_{t-1} + k_t
    for b in range(B):
        for h in range(H):
            St = torch.zeros(D, dv, dtype=F64)
            zt = torch.zeros(D, dtype=F64)
            for t in range(T):
                St = St + torch.outer(k[b, t, h], v[b, t, h])
                zt = zt + k[b, t, h]
                dn = max(scale * float(q[b, t, h] @ zt), eps)
                torch.testing.assert_close(den_d[b, t, h], torch.tensor(dn, dtype=F64))
                torch.testing.assert_close(o_d[b, t, h], scale * (q[b, t, h] @ St) / dn)
