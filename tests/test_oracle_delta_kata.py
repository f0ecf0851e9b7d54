"""Pins the SPD delta-rule oracle (``oracle/delta_kata.py``, the reference's
``flash_delta``, ``kata/spd/flash_delta.py:1060-1116``).  The reference holds
no outputs for it, so:

* the dense Gram / triangular-solve form equals the per-token delta rule on
  explicit E^2 features (two independent formulations);
* the sum-SPD Gram matches pure-Python loops at a tiny size;
* beta = 0 gives U = 0 and o = 0; a single token gives u = beta v and
  num = beta kappa(q, k) v;
* orthogonal features with beta kappa(k, k) = 1 overwrite exactly: the state
  read at k_i returns v_i;
* den is the row sum of tril(A_qk) and normalize divides by den + eps.
"""

import math

import pytest
import torch

from oracle import delta_kata as DK

F64 = torch.float64


def _rand(shape, seed, std=1.0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=F64) * std


@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("scale", [None, 0.5])
def test_dense_equals_feature_recurrence(M, scale):
    B, T, H, D, DV = 2, 23, 2, 8, 5
    q, k, v = _rand((B, T, H, D), 1, 0.5), _rand((B, T, H, D), 2, 0.5), _rand((B, T, H, DV), 3)
    beta = torch.sigmoid(_rand((B, T, H), 4))
    o, U, num, den = DK.flash_delta_fwd(q, k, v, beta, M, scale)
    num_r, S = DK.flash_delta_recurrent(q, k, v, beta, M, scale)
    torch.testing.assert_close(num, num_r, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(o, num)


def test_gram_brute_force():
    B, T, H, D, M = 1, 4, 1, 6, 3
    a, b = _rand((B, T, H, D), 5), _rand((B, T, H, D), 6)
    E, sc = D // M, 0.3
    G = DK.kappa_gram(a, b, M, sc)
    for t in range(T):
        for u in range(T):
            want = 0.0
            for g in range(M):
                for h in range(M):
                    d = sum(float(a[0, t, 0, g * E + e]) * float(b[0, u, 0, h * E + e]) for e in range(E))
                    want += (sc * d) ** 2
            assert float(G[0, 0, t, u]) == pytest.approx(want, rel=1e-12)


def test_beta_zero_and_single_token():
    B, T, H, D, DV, M = 1, 9, 2, 8, 3, 2
    q, k, v = _rand((B, T, H, D), 7), _rand((B, T, H, D), 8), _rand((B, T, H, DV), 9)
    o, U, num, den = DK.flash_delta_fwd(q, k, v, torch.zeros(B, T, H, dtype=F64), M)
    assert U.abs().max() == 0 and num.abs().max() == 0
    # one token: u = beta v, num = beta kappa(q, k) v
    beta = torch.sigmoid(_rand((B, 1, H), 10))
    o, U, num, den = DK.flash_delta_fwd(q[:, :1], k[:, :1], v[:, :1], beta, M)
    kap = DK.kappa_gram(q[:, :1], k[:, :1], M)[..., 0, 0]  # (B, H)
    torch.testing.assert_close(U, beta[..., None] * v[:, :1])
    torch.testing.assert_close(num, (beta * kap.unsqueeze(1))[..., None] * v[:, :1])
    torch.testing.assert_close(den, kap.unsqueeze(1))


def test_orthogonal_overwrite():
    # M = 1, E = 2, scale = 1: phi(e1) and phi(e2) are orthogonal unit features;
    # with beta = 1 each write replaces what the state returns for that key
    e1 = torch.tensor([1.0, 0.0], dtype=F64)
    e2 = torch.tensor([0.0, 1.0], dtype=F64)
    keys = torch.stack([e1, e2, e1, e2, e1])[None, :, None, :]
    v = _rand((1, 5, 1, 3), 11)
    beta = torch.ones(1, 5, 1, dtype=F64)
    num, S = DK.flash_delta_recurrent(keys, keys, v, beta, 1, scale=1.0)
    o, U, num_d, den = DK.flash_delta_fwd(keys, keys, v, beta, 1, scale=1.0)
    torch.testing.assert_close(num_d, num)
    # reading with q = the last key of each kind returns the latest value written for it
    torch.testing.assert_close(num_d[0, 4, 0], v[0, 4, 0])
    torch.testing.assert_close(num_d[0, 3, 0], v[0, 3, 0])


def test_normalize_and_den():
    B, T, H, D, DV, M = 1, 12, 1, 8, 4, 2
    q, k, v = _rand((B, T, H, D), 12), _rand((B, T, H, D), 13), _rand((B, T, H, DV), 14)
    beta = torch.sigmoid(_rand((B, T, H), 15))
    o, U, num, den = DK.flash_delta_fwd(q, k, v, beta, M, normalize=True, eps=1e-3)
    A = torch.tril(DK.kappa_gram(q, k, M))
    torch.testing.assert_close(den, A.sum(-1).permute(0, 2, 1))
    torch.testing.assert_close(o, num / (den[..., None] + 1e-3))


def test_gradients_gradcheck():
    """The oracle's autograd gradients (what the GPU backward is checked
    against) agree with finite differences on a tiny case, normalised too."""
    g = torch.Generator().manual_seed(4)
    B, T, H, D, M = 1, 5, 1, 8, 2
    q = torch.randn(B, T, H, D, generator=g, dtype=torch.float64) * 0.5
    k = torch.randn(B, T, H, D, generator=g, dtype=torch.float64) * 0.5
    v = torch.randn(B, T, H, 3, generator=g, dtype=torch.float64)
    beta = torch.rand(B, T, H, generator=g, dtype=torch.float64)
    for normalize in (False, True):
        f = lambda *a: DK.flash_delta_fwd(*a, M, 0.7, normalize)[0]  # noqa: E731
        ins = [t.clone().requires_grad_(True) for t in (q, k, v, beta)]
        assert torch.autograd.gradcheck(f, ins, eps=1e-6, atol=1e-6)


def test_dbeta_closed_form_at_beta_zero():
    """beta = 0: U = 0 and o = 0, so dq = dk = dv = 0 and, with dbV = dU =
    lower(A_qk)^T do, dbeta_t = <v_t, sum_{s >= t} A_qk[s, t] do_s>."""
    g = torch.Generator().manual_seed(6)
    B, T, H, D, M = 2, 9, 2, 8, 2
    q, k = (torch.randn(B, T, H, D, generator=g, dtype=torch.float64) for _ in range(2))
    v, do = (torch.randn(B, T, H, 4, generator=g, dtype=torch.float64) for _ in range(2))
    beta = torch.zeros(B, T, H, dtype=torch.float64)
    o, dq, dk, dv, db = DK.flash_delta_fwd_bwd(q, k, v, beta, M, do, 0.5)
    assert o.abs().max() == 0 and dq.abs().max() == 0 and dk.abs().max() == 0
    Aqk = torch.tril(DK.kappa_gram(q, k, M, 0.5))                  # (B, H, T, T)
    dU = torch.einsum("bhts,bthd->bshd", Aqk, do)
    assert torch.allclose(dv, beta[..., None] * dU)
    assert torch.allclose(db, (v * dU).sum(-1), atol=1e-12)
    # and the mistake of dropping the transpose fails
    wrong = torch.einsum("bhst,bthd->bshd", Aqk, do)
    assert not torch.allclose(db, (v * wrong).sum(-1), atol=1e-6)
