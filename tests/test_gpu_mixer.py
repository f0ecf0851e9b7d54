"""GPU parity of the mixer's short convolution, RMSNorm and rotary embedding
(``linatt_amd.mixer``, C ABI ``linatt_short_conv_*`` / ``linatt_rmsnorm_*`` /
``linatt_rope``)
against the float64 oracle ``oracle/mixer.py`` (forward and float64 autograd
gradients).  Inputs are drawn on the CPU, rounded once to the test dtype and
shared by both sides.  Metric ``max|x - ref| / max|ref|``; bars: float32
1e-5, bfloat16 2e-2, float16 1e-2."""

import pytest
import torch

from oracle import mixer as X

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 1e-2}
DT = [torch.bfloat16, torch.float16, torch.float32]


def mar(x, ref):
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = ref.abs().max().item()
    return (x - ref).abs().max().item() / (den if den > 0 else 1.0)


@pytest.fixture(scope="module")
def MX():
    from linatt_amd import mixer as MX
    return MX


def _conv_data(B, T, C, W, dtype, seed, bias, cache):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, C, generator=g).to(dtype)
    w = (torch.randn(C, 1, W, generator=g) / W).to(dtype)
    b = torch.randn(C, generator=g).to(dtype) if bias else None
    c = torch.randn(B, C, W, generator=g).to(dtype) if cache else None
    dy = torch.randn(B, T, C, generator=g).to(dtype)
    return x, w, b, c, dy


@pytest.mark.parametrize("shape", [(1, 1, 8), (2, 37, 64), (2, 300, 768), (1, 1000, 136)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("W", [2, 3, 4])
@pytest.mark.parametrize("act", ["silu", None])
@pytest.mark.parametrize("dtype", DT, ids=["bf16", "f16", "f32"])
def test_short_conv_parity(MX, shape, W, act, dtype):
    B, T, C = shape
    bias, cache = (W != 3), (W == 4)
    x, w, b, c, dy = _conv_data(B, T, C, W, dtype, T + W, bias, cache)
    print(f"\nshort_conv {shape} W={W} act={act} {dtype} bias={bias} cache={cache}", flush=True)
    ins = [x, w, b]
    y_ref, grads = X.fwd_bwd(lambda xx, ww, bb: X.short_conv(xx, ww, bb, act, c), ins, dy)
    _, fin_ref = X.short_conv(x, w, b, act, c)
    dev = torch.device("cuda")
    xd = x.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    bd = b.to(dev).requires_grad_(True) if b is not None else None
    y, fin = MX.short_conv(xd, wd, bd, act, c.to(dev) if c is not None else None,
                           output_final_state=True)
    y.backward(dy.to(dev))
    tol = TOL[dtype]
    assert mar(y, y_ref) < tol, ("y", mar(y, y_ref))
    assert torch.equal(fin.cpu(), fin_ref.to(dtype)), "final cache"
    for name, got, ref in (("dx", xd.grad, grads[0]), ("dw", wd.grad, grads[1]),
                           ("db", bd.grad if bd is not None else None, grads[2])):
        if ref is None:
            continue
        # float32 weight gradients sum B*T products: allow the summation order
        t = tol if dtype != torch.float32 or name == "dx" else 1e-4
        assert mar(got, ref) < t, (name, mar(got, ref))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_short_conv_decode_equals_full(MX, dtype):
    """Prefill then one-token steps through the cache reproduce the full
    sequence's outputs bit for bit (the same sums in the same order)."""
    B, T, C, W = 2, 40, 96, 4
    x, w, b, c, _ = _conv_data(B, T, C, W, dtype, 5, True, True)
    dev = torch.device("cuda")
    xd, wd, bd, cd = x.to(dev), w.to(dev), b.to(dev), c.to(dev)
    full, fin_full = MX.short_conv(xd, wd, bd, "silu", cd, output_final_state=True)
    n0 = 13
    outs = []
    y, st = MX.short_conv(xd[:, :n0], wd, bd, "silu", cd, output_final_state=True)
    outs.append(y)
    for t in range(n0, T):
        y, st = MX.short_conv(xd[:, t:t + 1], wd, bd, "silu", st, output_final_state=True)
        outs.append(y)
    assert torch.equal(torch.cat(outs, 1), full)
    assert torch.equal(st, fin_full)


def test_short_conv_module(MX):
    """The module: parameter names and shapes of nn.Conv1d, (y, cache) return."""
    torch.manual_seed(0)
    m = MX.ShortConvolution(64, 4, bias=False, activation="silu").cuda()
    assert m.weight.shape == (64, 1, 4) and m.bias is None
    assert set(dict(m.named_parameters())) == {"weight"}
    x = torch.randn(2, 50, 64, device="cuda")
    y, st = m(x, output_final_state=True)
    ref, fin = X.short_conv(x.cpu(), m.weight.detach().cpu(), None, "silu")
    assert mar(y, ref) < 1e-5 and st.shape == (2, 64, 4)
    y2, none = m(x)
    assert none is None and torch.equal(y2, y)
    with pytest.raises(NotImplementedError):
        m(x, cu_seqlens=torch.tensor([0, 50], device="cuda"))


@pytest.mark.parametrize("n,d", [(1, 64), (1000, 64), (4099, 128), (777, 8), (300, 512)])
@pytest.mark.parametrize("affine", [True, False])
@pytest.mark.parametrize("dtype", DT, ids=["bf16", "f16", "f32"])
def test_rmsnorm_parity(MX, n, d, affine, dtype):
    g = torch.Generator().manual_seed(n + d)
    x = (torch.randn(n, d, generator=g) * 2).to(dtype)
    w = torch.linspace(0.5, 1.5, d) if affine else None
    dy = torch.randn(n, d, generator=g).to(dtype)
    print(f"\nrmsnorm n={n} d={d} affine={affine} {dtype}", flush=True)
    y_ref, grads = X.fwd_bwd(lambda xx, ww: X.rmsnorm(xx, ww, 1e-5), [x, w], dy)
    dev = torch.device("cuda")
    xd = x.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True) if w is not None else None
    y = MX.rms_norm(xd, wd, 1e-5)
    assert y.dtype == dtype
    y.backward(dy.to(dev))
    tol = TOL[dtype]
    assert mar(y, y_ref) < tol, ("y", mar(y, y_ref))
    assert mar(xd.grad, grads[0]) < tol, ("dx", mar(xd.grad, grads[0]))
    if affine:
        t = tol if dtype != torch.float32 else 1e-4
        assert mar(wd.grad, grads[1]) < t, ("dw", mar(wd.grad, grads[1]))


def test_rmsnorm_module_on_heads(MX):
    """The mixer's output norm: (B, T, H, dv) bf16 with an fp32 weight."""
    m = MX.RMSNorm(64, elementwise_affine=True, eps=1e-5, dtype=torch.float32).cuda()
    with torch.no_grad():
        m.weight.copy_(torch.linspace(0.8, 1.2, 64))
    x = torch.randn(2, 33, 12, 64).bfloat16()
    y = m(x.cuda())
    assert y.shape == x.shape and y.dtype == torch.bfloat16
    assert mar(y, X.rmsnorm(x, m.weight.detach().cpu(), 1e-5)) < 2e-2


def test_repeat_runs_identical(MX):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4, 2048, 768, generator=g).bfloat16().cuda().requires_grad_(True)
    w = (torch.randn(768, 1, 4, generator=g) / 4).cuda().requires_grad_(True)
    dy = torch.randn(4, 2048, 768, generator=g).bfloat16().cuda()
    res = []
    for _ in range(3):
        x.grad = w.grad = None
        y, _ = MX.short_conv(x, w, None, "silu")
        y.backward(dy)
        res.append((y.detach().clone(), x.grad.clone(), w.grad.clone()))
    for r in res[1:]:
        for a, b in zip(r, res[0]):
            assert torch.equal(a, b)


@pytest.mark.parametrize("interleaved", [True, False], ids=["gptj", "neox"])
@pytest.mark.parametrize("dtype", DT, ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("shape,rot,offset", [((2, 300, 12, 64), 64, 0), ((1, 17, 3, 64), 48, 5),
                                              ((2, 50, 8, 16), 16, 2040),
                                              ((2, 40, 8, 96), 96, 3), ((1, 33, 5, 48), 32, 0)],
                         ids=["full", "partial", "group-late", "d96", "d48"])
def test_rope_parity(MX, interleaved, dtype, shape, rot, offset):
    """fwd against the float64 oracle; bwd = the inverse rotation of dy (the
    rotation is orthogonal), checked against float64 autograd."""
    g = torch.Generator().manual_seed(rot + offset)
    x = torch.randn(*shape, generator=g).to(dtype)
    dy = torch.randn(*shape, generator=g).to(dtype)
    y_ref, grads = X.fwd_bwd(lambda xx: X.rope(xx, rot, 10000.0, offset, interleaved), [x], dy)
    xd = x.cuda().requires_grad_(True)
    y = MX.rotary(xd, rot, 10000.0, offset, interleaved)
    y.backward(dy.cuda())
    # fp32: the angle (t + offset) * inv_freq is formed in fp32, as fla forms it
    # (pos_idx_in_fp32), so positions near 2048 carry ~1e-4 rad: the 1e-4 bar
    tol = 1e-4 if dtype == torch.float32 else TOL[dtype]
    assert mar(y, y_ref) < tol and mar(xd.grad, grads[0]) < tol


def test_rope_module_decode_offset(MX):
    """Decode through the module: token t with seqlen_offset t equals row t of
    the full-sequence rotation."""
    m = MX.RotaryEmbedding(64, base=10000.0, interleaved=True)
    q = torch.randn(1, 40, 4, 64, device="cuda").bfloat16()
    k = torch.randn(1, 40, 4, 64, device="cuda").bfloat16()
    qf, kf = m(q, k)
    for t in (0, 17, 39):
        qt, kt = m(q[:, t:t + 1], k[:, t:t + 1], seqlen_offset=t)
        assert torch.equal(qt, qf[:, t:t + 1]) and torch.equal(kt, kf[:, t:t + 1])
