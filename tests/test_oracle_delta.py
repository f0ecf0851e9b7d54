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
* finite differences (``gradcheck``) on the recurrence, incl. dg and dh0.
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
