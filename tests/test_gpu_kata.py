"""GPU parity of the HIP KATA kernels against the float64 CPU oracle.

Inputs are drawn on the CPU from seeded generators in float32, rounded once
to the test dtype, and the same rounded tensors feed both the GPU path and
(upcast) the oracle.  Error metric: max-abs-relative
``max|x - ref| / max|ref|`` per tensor; bars: float32 1e-4, bfloat16 2e-2,
float16 1e-2.  Every case calls the C ABI through ``linatt_amd``.
"""

import math

import pytest
import torch

from oracle import kata as K

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 1e-2}


def mar(x, ref, floor=0.0):
    """max|x - ref| / max(max|ref|, floor).  The floor matters only where the
    exact result vanishes identically (e.g. dq, dk at T=1, where o_0 = v_0 for
    any q, k): the oracle then returns ~1e-16 noise and the ratio would
    measure noise against noise."""
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = max(ref.abs().max().item(), floor)
    return (x - ref).abs().max().item() / (den if den > 0 else 1.0)


def grad_floors(q, k, v, do):
    """10% of the natural gradient scales: o is invariant to the scale of q
    (and of k), so |dq| ~ |dO||v|/|q| and |dk| ~ |dO||v|/|k|."""
    m = lambda t: t.detach().abs().max().item()  # noqa: E731
    return {"dq": 0.1 * m(do) * m(v) / m(q), "dk": 0.1 * m(do) * m(v) / m(k), "dv": 0.0}


def gen(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32) * std


@pytest.fixture(scope="module")
def P():
    from linatt_amd import parallel_kata_attn as P
    return P


def make(B, T, HQ, H, dk, dv, dtype, seed, std=0.125):
    q = gen((B, T, HQ, dk), seed, std).to(dtype)
    k = gen((B, T, H, dk), seed + 1, std).to(dtype)
    v = gen((B, T, H, dv), seed + 2, std).to(dtype)
    do = gen((B, T, HQ, dv), seed + 3, 1.0).to(dtype)
    return q, k, v, do


SHAPES = [  # B, T, HQ, H
    (1, 1, 1, 1),
    (2, 37, 2, 2),
    (1, 64, 1, 1),
    (1, 129, 3, 3),
    (2, 300, 2, 2),
    (1, 200, 4, 2),  # GQA
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("variant", ["concat", "sum"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16],
                         ids=["bf16", "f32", "f16"])
def test_fwd_bwd_parity(P, shape, M, variant, dtype):
    B, T, HQ, H = shape
    print(f"case {shape} M={M} {variant} {dtype}", flush=True)
    q, k, v, do = make(B, T, HQ, H, 64, 64, dtype, seed=100 + T + M)
    o_ref, den_ref = K.kata_fwd(q, k, v, M, None, variant)
    dq_ref, dk_ref, dv_ref = K.kata_bwd(q, k, v, o_ref, den_ref, do, M, None, variant)
    dev = torch.device("cuda")
    qd, kd, vd, dod = (x.to(dev) for x in (q, k, v, do))
    impl = P.parallel_kata_attn_fwd_impl if variant == "concat" else P.parallel_kata_attn_sum_fwd_impl
    o, den = impl(qd, kd, vd, M, 1 / math.sqrt(64 // M), 64, 64)
    assert o.dtype == dtype and den.dtype == torch.float32
    tol = TOL[dtype]
    eo, ed = mar(o, o_ref), mar(den, den_ref)
    assert eo < tol, ("o", eo)
    assert ed < tol, ("den", ed)
    bwd = P.parallel_kata_attn_bwd if variant == "concat" else P.parallel_kata_attn_bwd_sum
    dq, dk, dv = bwd(qd, kd, vd, o, den, dod, M, 1 / math.sqrt(64 // M))
    fl = grad_floors(q, k, v, do)
    for name, x, ref in (("dq", dq, dq_ref), ("dk", dk, dk_ref), ("dv", dv, dv_ref)):
        assert x.dtype == dtype
        e = mar(x, ref, fl[name])
        assert e < tol, (name, e)


@pytest.mark.parametrize("variant", ["concat", "sum"])
def test_autograd_function(P, variant):
    q, k, v, do = make(2, 150, 3, 3, 64, 64, torch.bfloat16, seed=7)
    dev = torch.device("cuda")
    leaves = [x.to(dev).requires_grad_(True) for x in (q, k, v)]
    fn = P.parallel_kata_attn if variant == "concat" else P.parallel_kata_attn_sum
    o = fn(*leaves, num_groups=4)
    o.backward(do.to(dev))
    o_ref, den_ref = K.kata_fwd(q, k, v, 4, None, variant)
    refs = K.kata_bwd(q, k, v, o_ref, den_ref, do, 4, None, variant)
    assert mar(o, o_ref) < 2e-2
    for leaf, ref in zip(leaves, refs):
        assert leaf.grad.dtype == torch.bfloat16
        assert mar(leaf.grad, ref) < 2e-2


@pytest.mark.parametrize("M", [1, 2, 4])
def test_config1_fp32(P, M):
    """fp32 (1,4,512,64) head-major q,k,v ~ N(0,1), seed 0."""
    g = torch.Generator().manual_seed(0)
    qh, kh, vh = (torch.randn(1, 4, 512, 64, generator=g) for _ in range(3))
    q, k, v = (x.transpose(1, 2).contiguous() for x in (qh, kh, vh))
    o_ref, den_ref = K.kata_fwd(q, k, v, M)
    o, den = P.parallel_kata_attn_fwd(q.cuda(), k.cuda(), v.cuda(), num_groups=M)
    assert o.transpose(1, 2).shape == (1, 4, 512, 64)
    assert mar(o, o_ref) < 1e-4
    assert mar(den, den_ref) < 1e-4


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_decay_forward(P, dtype):
    B, T, H = 2, 190, 3
    q, k, v, _ = make(B, T, H, H, 64, 64, dtype, seed=21)
    g = torch.Generator().manual_seed(22)
    c = -torch.cumsum(torch.rand(B, T, H, generator=g) * 0.1, dim=1)
    o_ref, den_ref = K.kata_fwd(q, k, v, 2, None, "concat", c=c)
    o, den = P.parallel_kata_attn_fwd_impl(q.cuda(), k.cuda(), v.cuda(), 2, None, 64, 64, c=c.cuda())
    assert mar(o, o_ref) < TOL[dtype]
    assert mar(den, den_ref) < TOL[dtype]


@pytest.mark.parametrize("M", [4, 2, 1])
def test_config2_full_size(P, M):
    """BASELINE config 2 at full size: B8 H12 T2048 D64 bf16, q,k,v ~ N(0,1)/8,
    dO ~ N(0,1), seed 1.  Two heads are compared with the float64 oracle; the
    whole output is checked through size-independent identities:
    sum_s dV[s] = sum_t dO[t] (rows of P sum to one), and <dq_t, q_t> = 0 and
    sum_s <dk_s, k_s> = 0 per head (o is invariant to rescaling q_t, or all k).
    """
    B, T, H, D = 8, 2048, 12, 64
    g = torch.Generator().manual_seed(1)
    q, k, v = ((torch.randn(B, T, H, D, generator=g) / 8).to(torch.bfloat16) for _ in range(3))
    do = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16)
    dev = torch.device("cuda")
    leaves = [x.to(dev).requires_grad_(True) for x in (q, k, v)]
    o = P.parallel_kata_attn(*leaves, num_groups=M)
    o.backward(do.to(dev))
    dq, dk, dv = (x.grad for x in leaves)
    for b, h in ((0, 0), (7, 11), (3, 5)):
        sl = lambda x: x[b:b + 1, :, h:h + 1]  # noqa: E731
        o_ref, den_ref = K.kata_fwd(sl(q), sl(k), sl(v), M)
        refs = K.kata_bwd(sl(q), sl(k), sl(v), o_ref, den_ref, sl(do), M)
        e = mar(sl(o), o_ref)
        assert e < 2e-2, ("o", b, h, e)
        for name, x, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), refs):
            e = mar(sl(x), ref)
            assert e < 2e-2, (name, b, h, e)
    dof = do.to(dev).float()
    lhs = dv.float().sum(1)
    rhs = dof.sum(1)
    assert (lhs - rhs).abs().max().item() / rhs.abs().max().item() < 2e-2
    # rows whose exact gradient is zero carry only rounding noise, so the
    # identities are normalised by the largest |dq_t||q_t| (resp. per-head sum)
    qd = (dq.float() * leaves[0].detach().float()).sum(-1)
    nq = (dq.float().norm(dim=-1) * leaves[0].detach().float().norm(dim=-1))
    assert qd.abs().max().item() / nq.max().item() < 2e-2
    kd = (dk.float() * leaves[1].detach().float()).sum((1, 3))
    nk = (dk.float().norm(dim=-1) * leaves[1].detach().float().norm(dim=-1)).sum(1)
    assert kd.abs().max().item() / nk.max().item() < 2e-2
    assert torch.isfinite(dq).all() and torch.isfinite(dk).all() and torch.isfinite(dv).all()


def test_deterministic(P):
    q, k, v, do = make(2, 333, 2, 2, 64, 64, torch.bfloat16, seed=31)
    dev = torch.device("cuda")
    outs = []
    for _ in range(2):
        o, den = P.parallel_kata_attn_fwd(q.to(dev), k.to(dev), v.to(dev))
        grads = P.parallel_kata_attn_bwd(q.to(dev), k.to(dev), v.to(dev), o, den, do.to(dev), 4, 0.25)
        outs.append((o, den) + grads)
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("shape", [(1, 1, 1), (2, 37, 2), (1, 190, 3), (2, 300, 2)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("cmode", ["cumulative", "arbitrary"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_decay_fwd_bwd(P, shape, M, cmode, dtype):
    """Decayed concat score (reference _KataDecayFunction, parallel_kata_attn.py:313-354):
    o, dq, dk, dv and dc against float64 autograd through the restated
    _kata_decay_ref.  'cumulative' c is a running sum of log decays (the
    layer's use, kata/layer.py:440-447); 'arbitrary' c exercises the
    min(c_t - c_s, 0) clamp and its gradient mask."""
    B, T, H = shape
    q, k, v, do = make(B, T, H, H, 64, 64, dtype, seed=40 + T + M)
    g = torch.Generator().manual_seed(41 + T)
    if cmode == "cumulative":
        c = -torch.cumsum(torch.rand(B, T, H, generator=g) * 0.1, dim=1)
    else:
        c = torch.randn(B, T, H, generator=g) * 0.5
    o_ref, dq_ref, dk_ref, dv_ref, dc_ref = K.kata_decay_fwd_bwd(q, k, v, c, do, M)
    dev = torch.device("cuda")
    leaves = [x.to(dev).requires_grad_(True) for x in (q, k, v, c)]
    o = P.parallel_kata_attn_decay(*leaves, num_groups=M)
    o.backward(do.to(dev))
    tol = TOL[dtype]
    assert mar(o, o_ref) < tol
    fl = grad_floors(q, k, v, do)
    fl["dc"] = 0.1 * do.abs().max().item() * v.abs().max().item()
    for name, leaf, ref in zip(("dq", "dk", "dv", "dc"), leaves, (dq_ref, dk_ref, dv_ref, dc_ref)):
        assert leaf.grad.dtype == leaf.dtype
        e = mar(leaf.grad, ref, fl[name])
        assert e < tol, (name, e)


def _augment_offset(q, k, off, M, E, Ep):
    """The offset-gated mixer's packing (kata/layer.py:265-281): per group, q
    gets [q_g, off_t, 0...] and k gets [k_g, 1, 0...], each padded to Ep, so
    the concat score becomes sum_g (scale (q_g . k_g + off_t))^2."""
    B, T, H, _ = q.shape

    def pack(x, col):
        xg = x.reshape(B, T, H, M, E)
        cc = col[..., None, None].expand(B, T, H, M, 1).to(x.dtype)
        z = x.new_zeros(B, T, H, M, Ep - E - 1)
        return torch.cat([xg, cc, z], dim=-1).reshape(B, T, H, M * Ep)

    return pack(q, off), pack(k, torch.ones_like(off))


@pytest.mark.parametrize("decay", [False, True], ids=["plain", "decay"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("T", [200, 333])
def test_offset_gate_shape_dk128(P, decay, dtype, T):
    """dk = 128, dv = 64, M = 2: the shape kataconv_cat_l2_gdn_340m.yaml:12,18-19
    runs (M = 2 groups of E = 32 padded to 64 by the offset gate; scale =
    1/sqrt(32) passed explicitly, kata/layer.py:237-244, 440-455)."""
    B, H, M, E, Ep, dv = 2, 2, 2, 32, 64, 64
    q0 = gen((B, T, H, M * E), 60 + T, 0.125)
    k0 = gen((B, T, H, M * E), 61 + T, 0.125)
    off = torch.sigmoid(gen((B, T, H), 62 + T))
    q, k = _augment_offset(q0, k0, off, M, E, Ep)
    q, k = q.to(dtype), k.to(dtype)
    v = gen((B, T, H, dv), 63 + T, 0.125).to(dtype)
    do = gen((B, T, H, dv), 64 + T).to(dtype)
    scale = 1.0 / math.sqrt(E)
    dev = torch.device("cuda")
    tol = TOL[dtype]
    if decay:
        c = -torch.cumsum(torch.rand(B, T, H, generator=torch.Generator().manual_seed(65)) * 0.1, 1)
        o_ref, *grads_ref = K.kata_decay_fwd_bwd(q, k, v, c, do, M, scale)
        leaves = [x.to(dev).requires_grad_(True) for x in (q, k, v, c)]
        o = P.parallel_kata_attn_decay(*leaves, num_groups=M, scale=scale)
        names = ("dq", "dk", "dv", "dc")
    else:
        o_ref, den_ref = K.kata_fwd(q, k, v, M, scale)
        grads_ref = K.kata_bwd(q, k, v, o_ref, den_ref, do, M, scale)
        leaves = [x.to(dev).requires_grad_(True) for x in (q, k, v)]
        o = P.parallel_kata_attn(*leaves, num_groups=M, scale=scale)
        names = ("dq", "dk", "dv")
    o.backward(do.to(dev))
    assert mar(o, o_ref) < tol
    fl = grad_floors(q, k, v, do)
    fl["dc"] = 0.1 * do.abs().max().item() * v.abs().max().item()
    for name, leaf, ref in zip(names, leaves, grads_ref):
        e = mar(leaf.grad, ref, fl[name])
        assert e < tol, (name, e)
    # the zero padding of every group receives gradient only through the
    # offset coordinate: the padded columns of dq, dk stay (numerically) zero
    if not decay:
        pad = leaves[0].grad.reshape(B, T, H, M, Ep)[..., E + 1:]
        assert pad.abs().max().item() <= 1e-6 * max(1.0, leaves[0].grad.abs().max().item())


@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (2, 37, 2, 2), (1, 300, 2, 2), (1, 520, 4, 2)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("variant", ["concat", "sum", "decay"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32],
                         ids=["bf16", "f16", "f32"])
def test_dense_dk128(P, shape, variant, dtype):
    """dk = 128, dv = 64, M = 2 with every key column live (the offset gate's
    inputs leave half of each group zero): one key block, two and three
    blocks of 256 keys with a ragged end, and GQA (HQ = 2 H)."""
    B, T, HQ, H = shape
    M = 2
    print(f"case {shape} dk128 {variant} {dtype}", flush=True)
    q, k, v, do = make(B, T, HQ, H, 128, 64, dtype, seed=300 + T)
    dev = torch.device("cuda")
    tol = TOL[dtype]
    fl = grad_floors(q, k, v, do)
    if variant == "decay":
        c = -torch.cumsum(torch.rand(B, T, HQ, generator=torch.Generator().manual_seed(T)) * 0.1, 1)
        # GQA: the oracle's decayed form over k, v repeated to the query heads
        # (query head hq reads kv head hq // G); dk, dv of a kv head are the
        # sums over its G query heads
        G = HQ // H
        o_ref, dq_r, dk_r, dv_r, dc_r = K.kata_decay_fwd_bwd(
            q, k.repeat_interleave(G, dim=2), v.repeat_interleave(G, dim=2), c, do, M)
        refs = (dq_r, dk_r.reshape(B, T, H, G, -1).sum(3), dv_r.reshape(B, T, H, G, -1).sum(3), dc_r)
        leaves = [x.to(dev).requires_grad_(True) for x in (q, k, v, c)]
        o = P.parallel_kata_attn_decay(*leaves, num_groups=M)
        names = ("dq", "dk", "dv", "dc")
        fl["dc"] = 0.1 * do.abs().max().item() * v.abs().max().item()
    else:
        o_ref, den_ref = K.kata_fwd(q, k, v, M, None, variant)
        refs = K.kata_bwd(q, k, v, o_ref, den_ref, do, M, None, variant)
        leaves = [x.to(dev).requires_grad_(True) for x in (q, k, v)]
        fn = P.parallel_kata_attn if variant == "concat" else P.parallel_kata_attn_sum
        o = fn(*leaves, num_groups=M)
        names = ("dq", "dk", "dv")
    o.backward(do.to(dev))
    assert mar(o, o_ref) < tol
    for name, leaf, ref in zip(names, leaves, refs):
        e = mar(leaf.grad, ref, fl[name])
        assert e < tol, (name, e)
