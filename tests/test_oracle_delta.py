"""Pins the delta-rule oracle (``oracle/delta.py``).

The reference holds no delta-rule outputs (the arithmetic lives in the absent
third-party ``fla`` package), so the oracle is pinned by mathematics:

* the chunked WY/UT form equals the naive per-token recurrence (forward, final
  state and every gradient), for ragged T, T < C, T == C, several chunks;
* beta == 0 freezes the state: o = scale * q^T h0 (gates still decay it);
* g == 0 reduces GatedDeltaNet to DeltaNet;
* with orthonormal keys and beta == 1 each write overwrites exactly:
  S^T k_i == v_i afterwards;
* a single step from S=0 gives o = scale * beta (q.k) v (closed form);
* finite differences (``gradcheck``) on the recurrence, incl. dg and dh0;
* gated with beta == 0: S_T = e^{sum g} h0 and o_t = scale e^{G_t} h0^T q_t;
* l2norm by closed forms: unit rows, direction and scale invariance, and the
  eps placement inside the square root (x / sqrt(x^2 + eps) for one element).
"""

import math

import pytest
import torch

from oracle import delta as D

F64 = torch.float64


def _inputs(B, T, H, K, V, seed, gated=True, h0=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=g, dtype=F64)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=g, dtype=F64), dim=-1)
    v = torch.randn(B, T, H, V, generator=g, dtype=F64)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g, dtype=F64))
    gg = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=g, dtype=F64) + 1.0) / 4 if gated else None
    s0 = torch.randn(B, H, K, V, generator=g, dtype=F64) * 0.1 if h0 else None
    return q, k, v, beta, gg, s0


@pytest.mark.parametrize("T,C", [(5, 8), (8, 8), (19, 8), (64, 16), (33, 64)])
@pytest.mark.parametrize("gated", [False, True])
def test_chunked_equals_recurrent(T, C, gated):
    q, k, v, beta, g, h0 = _inputs(2, T, 2, 6, 5, 1 + T, gated)
    o1, s1 = D.delta_rule_recurrent(q, k, v, beta, g, initial_state=h0)
    o2, s2 = D.delta_rule_chunked(q, k, v, beta, g, initial_state=h0, chunk=C)
    torch.testing.assert_close(o1, o2, rtol=1e-10, atol=1e-11)
    torch.testing.assert_close(s1, s2, rtol=1e-10, atol=1e-11)


@pytest.mark.parametrize("gated", [False, True])
def test_gradients_chunked_equal_recurrent(gated):
    q, k, v, beta, g, h0 = _inputs(1, 21, 2, 4, 3, 77, gated)
    gen = torch.Generator().manual_seed(5)
    do = torch.randn(1, 21, 2, 3, generator=gen, dtype=F64)
    dht = torch.randn(1, 2, 4, 3, generator=gen, dtype=F64)
    a = D.delta_rule_fwd_bwd(q, k, v, beta, g, initial_state=h0, do=do, dht=dht, chunk=8)
    b = D.delta_rule_fwd_bwd(q, k, v, beta, g, initial_state=h0, do=do, dht=dht, form="recurrent")
    assert set(a) == set(b)
    for key in a:
        torch.testing.assert_close(a[key], b[key], rtol=1e-9, atol=1e-10)


def test_beta_zero_freezes_state():
    q, k, v, beta, g, h0 = _inputs(2, 9, 2, 4, 3, 3, gated=False)
    o, s = D.delta_rule_recurrent(q, k, v, torch.zeros_like(beta), None, initial_state=h0)
    torch.testing.assert_close(s, h0)
    torch.testing.assert_close(o, torch.einsum("bthk,bhkv->bthv", q, h0) / 2.0)


def test_gate_zero_is_deltanet():
    q, k, v, beta, g, h0 = _inputs(1, 13, 2, 4, 3, 4, gated=True)
    a = D.delta_rule_recurrent(q, k, v, beta, torch.zeros_like(g), initial_state=h0)
    b = D.delta_rule_recurrent(q, k, v, beta, None, initial_state=h0)
    torch.testing.assert_close(a[0], b[0])
    torch.testing.assert_close(a[1], b[1])
    c = D.delta_rule_chunked(q, k, v, beta, torch.zeros_like(g), initial_state=h0, chunk=4)
    torch.testing.assert_close(a[0], c[0])


def test_orthonormal_keys_overwrite():
    Kd, V = 6, 4
    Qm, _ = torch.linalg.qr(torch.randn(Kd, Kd, generator=torch.Generator().manual_seed(9), dtype=F64))
    k = Qm.T[None, :, None, :]  # 6 orthonormal keys (B=1,T=6,H=1,K)
    v = torch.randn(1, Kd, 1, V, generator=torch.Generator().manual_seed(10), dtype=F64)
    h0 = torch.randn(1, 1, Kd, V, generator=torch.Generator().manual_seed(11), dtype=F64)
    beta = torch.ones(1, Kd, 1, dtype=F64)
    _, s = D.delta_rule_recurrent(k, k, v, beta, None, initial_state=h0)
    for i in range(Kd):
        torch.testing.assert_close(s[0, 0].T @ k[0, i, 0], v[0, i, 0])


def test_single_step_closed_form():
    q, k, v, beta, _, _ = _inputs(2, 1, 3, 8, 5, 12, gated=False, h0=False)
    o, s = D.delta_rule_recurrent(q, k, v, beta)
    want = (beta[..., None] * (q * k).sum(-1, keepdim=True) * v) / math.sqrt(8)
    torch.testing.assert_close(o, want)


def test_finite_differences():
    q, k, v, beta, g, h0 = _inputs(1, 5, 1, 3, 2, 13, gated=True)
    args = tuple(x.clone().requires_grad_(True) for x in (q, k, v, beta, g, h0))

    def f(q, k, v, beta, g, h0):
        o, s = D.delta_rule_recurrent(q, k, v, beta, g, initial_state=h0)
        return o.sum() + (s * s).sum()

    assert torch.autograd.gradcheck(f, args)


def test_l2norm_in_kernel():
    q, k, v, beta, g, h0 = _inputs(1, 10, 2, 4, 3, 14, gated=True)
    a = D.delta_rule_recurrent(q * 3, k * 2, v, beta, g, initial_state=h0, use_qk_l2norm=True)
    b = D.delta_rule_recurrent(D.l2norm(q * 3), D.l2norm(k * 2), v, beta, g, initial_state=h0)
    torch.testing.assert_close(a[0], b[0])
    c = D.delta_rule_chunked(q * 3, k * 2, v, beta, g, initial_state=h0, chunk=4, use_qk_l2norm=True)
    torch.testing.assert_close(a[0], c[0])


# ---------------------------------------------------------------------------
# l2norm: fla.modules.l2norm.l2norm (third-party, absent; called at
# kata/layer.py:347-348 and by use_qk_l2norm_in_kernel) is x / sqrt(sum x^2 + eps)
# with eps = 1e-6 inside the square root.  Pinned by closed forms.
# ---------------------------------------------------------------------------


def test_l2norm_closed_forms():
    x = torch.randn(7, 33, generator=torch.Generator().manual_seed(60), dtype=F64) * 5
    y = D.l2norm(x)
    # unit rows when |x|^2 >> eps
    torch.testing.assert_close(y.norm(dim=-1), torch.ones(7, dtype=F64), rtol=1e-6, atol=0)
    # direction kept: y is a positive multiple of x
    ratio = y / x
    torch.testing.assert_close(ratio, ratio[:, :1].expand_as(ratio))
    assert (ratio > 0).all()
    # scale invariance for large rows
    torch.testing.assert_close(D.l2norm(x * 1e3), y, rtol=1e-9, atol=1e-12)
    # eps inside the sqrt: a one-element row gives x / sqrt(x^2 + eps) exactly
    for xv in (1e-4, 3e-3, 0.5, -2.0):
        got = D.l2norm(torch.tensor([[xv]], dtype=F64)).item()
        assert got == pytest.approx(xv / math.sqrt(xv * xv + 1e-6), rel=1e-14)
    # eps placement distinguishes the plausible mistake x / (|x| + eps):
    # for |x| = 1e-4, inside -> ~0.0995, outside -> ~0.99
    small = torch.full((1, 4), 5e-5, dtype=F64)  # |x| = 1e-4
    assert D.l2norm(small).norm().item() == pytest.approx(1e-4 / math.sqrt(1e-8 + 1e-6), rel=1e-12)
    # a zero row stays zero (no division by zero)
    assert torch.equal(D.l2norm(torch.zeros(2, 5, dtype=F64)), torch.zeros(2, 5, dtype=F64))
    # explicit eps argument
    assert D.l2norm(torch.tensor([[0.1]], dtype=F64), eps=0.03).item() == pytest.approx(0.1 / math.sqrt(0.04), rel=1e-14)


# ---------------------------------------------------------------------------
# Gated rule with beta == 0: only the gate acts, S_t = e^{G_t} h0 with
# G_t = sum_{i<=t} g_i, so o_t = scale e^{G_t} h0^T q_t and S_T = e^{G_T} h0.
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("chunk", [None, 4, 8])
def test_gated_beta_zero_closed_form(chunk):
    q, k, v, beta, g, h0 = _inputs(2, 11, 3, 5, 4, 61, gated=True)
    beta0 = torch.zeros_like(beta)
    scale = 0.37
    if chunk is None:
        o, s = D.delta_rule_recurrent(q, k, v, beta0, g, scale=scale, initial_state=h0)
    else:
        o, s = D.delta_rule_chunked(q, k, v, beta0, g, scale=scale, initial_state=h0, chunk=chunk)
    G = torch.cumsum(g, 1)  # (B, T, H)
    want_o = scale * torch.exp(G)[..., None] * torch.einsum("bthk,bhkv->bthv", q, h0)
    want_s = torch.exp(G[:, -1])[..., None, None] * h0
    torch.testing.assert_close(o, want_o, rtol=1e-11, atol=1e-12)
    torch.testing.assert_close(s, want_s, rtol=1e-11, atol=1e-12)
    # a plausible mistake (decaying after the write instead of before, i.e.
    # G shifted by one step) is visible
    Gs = torch.cumsum(torch.cat([torch.zeros_like(g[:, :1]), g[:, :-1]], 1), 1)
    wrong = scale * torch.exp(Gs)[..., None] * torch.einsum("bthk,bhkv->bthv", q, h0)
    assert (wrong - o).abs().max() > 1e-3
