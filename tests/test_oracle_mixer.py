"""Pins for ``oracle/mixer.py`` (the mixer's short convolution and RMSNorm):
explicit loops, the library convolution, cache continuation and closed forms.
CPU only."""

import pytest
import torch

from oracle import mixer as X


def _data(B, T, C, W, seed, bias=True, cache=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, C, generator=g, dtype=torch.float64)
    w = torch.randn(C, W, generator=g, dtype=torch.float64) / W
    b = torch.randn(C, generator=g, dtype=torch.float64) if bias else None
    c = torch.randn(B, C, W, generator=g, dtype=torch.float64) if cache else None
    return x, w, b, c


@pytest.mark.parametrize("W", [2, 3, 4])
@pytest.mark.parametrize("act", ["silu", None])
@pytest.mark.parametrize("bias,cache", [(True, True), (False, False), (False, True)])
def test_conv_matches_loops(W, act, bias, cache):
    x, w, b, c = _data(2, 7, 5, W, W, bias, cache)
    y, _ = X.short_conv(x, w, b, act, c)
    assert torch.allclose(y, X.short_conv_loop(x, w, b, act, c), atol=1e-12)


@pytest.mark.parametrize("W", [2, 4])
def test_conv_matches_library_conv1d(W):
    """Without a cache: a depthwise nn.functional.conv1d with W - 1 left
    padding, truncated to T (the nn.Conv1d fla's module derives from)."""
    x, w, b, _ = _data(3, 20, 6, W, 11)
    ref = torch.nn.functional.conv1d(x.transpose(1, 2), w[:, None, :], b, padding=W - 1,
                                     groups=6)[..., :20].transpose(1, 2)
    y, _ = X.short_conv(x, w, b, None)
    assert torch.allclose(y, ref, atol=1e-12)
    ys, _ = X.short_conv(x, w[:, None, :], b, "silu")  # (C, 1, W) weights accepted
    assert torch.allclose(ys, ref * torch.sigmoid(ref), atol=1e-12)


@pytest.mark.parametrize("split", [1, 2, 3, 9])
def test_conv_cache_continuation(split):
    """A sequence cut anywhere, the second part continued from the first
    part's final cache, gives the same outputs and the same final cache."""
    x, w, b, c = _data(2, 12, 4, 4, 5)
    y, fin = X.short_conv(x, w, b, "silu", c)
    y1, f1 = X.short_conv(x[:, :split], w, b, "silu", c)
    y2, f2 = X.short_conv(x[:, split:], w, b, "silu", f1)
    assert torch.allclose(torch.cat([y1, y2], 1), y, atol=1e-12)
    assert torch.allclose(f2, fin, atol=0)
    # the final cache is the last W inputs, newest last
    assert torch.equal(fin, x[:, -4:].transpose(1, 2))


def test_conv_cache_shorter_sequence():
    """T < W: the final cache keeps the older cache entries before x."""
    x, w, b, c = _data(1, 2, 3, 4, 6)
    _, fin = X.short_conv(x, w, b, "silu", c)
    assert torch.equal(fin[:, :, :2], c[:, :, 2:])
    assert torch.equal(fin[:, :, 2:], x.transpose(1, 2))


def test_rmsnorm_closed_forms():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 64, generator=g, dtype=torch.float64) * 3
    eps = 1e-5
    y = X.rmsnorm(x, None, eps)
    ms = (x * x).mean(-1)
    assert torch.allclose((y * y).mean(-1), ms / (ms + eps), atol=1e-12)
    # scale invariance at eps = 0, weight scales each column
    assert torch.allclose(X.rmsnorm(7.5 * x, None, 0.0), X.rmsnorm(x, None, 0.0), atol=1e-12)
    w = torch.linspace(0.5, 2.0, 64, dtype=torch.float64)
    assert torch.allclose(X.rmsnorm(x, w, eps), y * w, atol=1e-12)
    # a constant row maps to sign * sqrt(c^2 / (c^2 + eps))
    c = torch.full((1, 64), -0.01, dtype=torch.float64)
    assert torch.allclose(X.rmsnorm(c, None, eps), -torch.full_like(c, (1e-4 / (1e-4 + eps)) ** 0.5))


@pytest.mark.parametrize("interleaved", [True, False])
def test_rope_relative_position(interleaved):
    """<R_t q, R_s k> depends on t - s only (per rotated pair), rotation keeps
    norms, the inverse undoes it, and dims past rot_dim pass through."""
    g = torch.Generator().manual_seed(2)
    D, rot = 16, 12
    q = torch.randn(1, 1, 1, D, generator=g, dtype=torch.float64).expand(1, 9, 1, D).contiguous()
    k = torch.randn(1, 1, 1, D, generator=g, dtype=torch.float64).expand(1, 9, 1, D).contiguous()
    rq, rk = X.rope(q, rot, 500.0, 0, interleaved), X.rope(k, rot, 500.0, 0, interleaved)
    dots = torch.einsum("btd,bsd->bts", rq[:, :, 0], rk[:, :, 0])
    for dlt in range(-3, 4):
        diag = torch.diagonal(dots, offset=dlt, dim1=1, dim2=2)
        assert torch.allclose(diag, diag[:, :1].expand_as(diag), atol=1e-12)
    assert torch.allclose(rq.norm(dim=-1), q.norm(dim=-1), atol=1e-12)
    assert torch.equal(rq[..., rot:], q[..., rot:])
    assert torch.allclose(X.rope(rq, rot, 500.0, 0, interleaved, inverse=True), q, atol=1e-12)
    # an offset is a shift in time
    assert torch.allclose(X.rope(q[:, 3:], rot, 500.0, 3, interleaved), rq[:, 3:], atol=1e-12)


def test_rope_layouts_are_a_permutation():
    """Interleaved pairs (2p, 2p+1) are the half-split pairs (p, p + D/2)
    after the matching permutation of the dims."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 5, 3, 8, generator=g, dtype=torch.float64)
    perm = torch.tensor([0, 4, 1, 5, 2, 6, 3, 7])  # interleaved dim -> half-split dim
    a = X.rope(x, 8, 100.0, 2, interleaved=True)
    b = X.rope(x[..., perm.argsort()], 8, 100.0, 2, interleaved=False)[..., perm]
    assert torch.allclose(a, b, atol=1e-12)


@pytest.mark.parametrize("interleaved", [True, False])
@pytest.mark.parametrize("offset", [0, 5])
def test_rope_closed_form_frequencies_and_sign(interleaved, offset):
    """RoFormer's rotation (Su et al. 2021, eq. 34) at single positions and
    pairs: pair p of a rot_dim-wide rotation at position t turns (a, b) into
    (a cos t th_p - b sin t th_p, a sin t th_p + b cos t th_p) with
    th_p = base^(-2p / rot_dim).  Checked element by element with scalar
    math at t = 1 and t = 7 (plus an offset) for the first and last pair, and
    against hand-computed constants for unit inputs."""
    import math
    g = torch.Generator().manual_seed(9)
    D, rot, base = 12, 8, 10000.0
    half = rot // 2
    x = torch.randn(1, 8, 1, D, generator=g, dtype=torch.float64)
    y = X.rope(x, rot, base, offset, interleaved)
    for t in (1, 7):
        pos = t + offset
        for p in (0, half - 1):
            i0, i1 = (2 * p, 2 * p + 1) if interleaved else (p, p + half)
            th = base ** (-2.0 * p / rot)
            a, b = float(x[0, t, 0, i0]), float(x[0, t, 0, i1])
            c, s = math.cos(pos * th), math.sin(pos * th)
            assert abs(float(y[0, t, 0, i0]) - (a * c - b * s)) < 1e-12
            assert abs(float(y[0, t, 0, i1]) - (a * s + b * c)) < 1e-12
    # unit vector on the first element of pair 1 at t = 7, rot_dim = 4,
    # base = 10000: th_1 = 10000^(-1/2) = 0.01, so the angle is 0.07 rad
    # and the rotated vector is (cos 0.07, sin 0.07) = (0.99755100, 0.06994285)
    e = torch.zeros(1, 8, 1, 4, dtype=torch.float64)
    i0, i1 = (2, 3) if interleaved else (1, 3)
    e[0, 7, 0, i0] = 1.0
    r = X.rope(e, 4, 10000.0, 0, interleaved)
    assert abs(float(r[0, 7, 0, i0]) - 0.9975510002532796) < 1e-12
    assert abs(float(r[0, 7, 0, i1]) - 0.0699428473375328) < 1e-12
    # pair 0 turns by t radians: at t = 1, (0, 1) -> (-sin 1, cos 1)
    e = torch.zeros(1, 2, 1, 4, dtype=torch.float64)
    j0, j1 = (0, 1) if interleaved else (0, 2)
    e[0, 1, 0, j1] = 1.0
    r = X.rope(e, 4, 10000.0, 0, interleaved)
    assert abs(float(r[0, 1, 0, j0]) + 0.8414709848078965) < 1e-12
    assert abs(float(r[0, 1, 0, j1]) - 0.5403023058681398) < 1e-12
