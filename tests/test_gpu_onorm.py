"""GPU parity of the mixer's output RMSNorm fused into the KATA kernels
(``linatt_kata_fwd_onorm`` / ``linatt_kata_bwd_onorm`` through
``parallel_kata_attn_onorm``) against the float64 oracle: KATA scores
(``oracle.kata.kata_fwd``) then ``oracle.mixer.rmsnorm``, with gradients by
float64 autograd for q, k, v, the norm weight and the decay's c.

Bars: bf16 2e-2 max-abs-relative per tensor (fp16 forward 1e-2).  Also: the
fused forward's o and den equal the plain forward's bit for bit, and the
fused output and gradients agree with the unfused HIP chain (KATA op, then
the standalone RMSNorm kernels) to within one rounding of each.
"""

import pytest
import torch

from oracle import kata as K
from oracle import mixer as X

pytestmark = pytest.mark.gpu
BAR = {torch.bfloat16: 2e-2, torch.float16: 1e-2}


def mar(x, ref, floor=0.0):
    """max|x - ref| / max(max|ref|, floor); the floor matters where the exact
    gradient vanishes (dq, dk at T = 1: o_0 = v_0 for any q, k)."""
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = max(ref.abs().max().item(), floor)
    return (x - ref).abs().max().item() / (den if den > 0 else 1.0)


def gen(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * std


@pytest.fixture(scope="module")
def P():
    from linatt_amd import parallel_kata_attn as P
    return P


def inputs(B, T, HQ, H, M, seed, dtype=torch.bfloat16, decay=False):
    D = 64
    q = gen((B, T, HQ, D), seed, 0.5).to(dtype)
    k = gen((B, T, H, D), seed + 1, 0.5).to(dtype)
    v = gen((B, T, H, D), seed + 2, 1.0).to(dtype)
    dy = gen((B, T, HQ, D), seed + 3).to(dtype)
    w = 0.75 + 0.5 * torch.rand(D, generator=torch.Generator().manual_seed(seed + 4))
    c = None
    if decay:
        lam = gen((B, T, HQ), seed + 5).abs() * 0.05
        c = (-lam).cumsum(1)
    return q, k, v, dy, w, c


def oracle(q, k, v, w, c, dy, M, variant, eps=1e-5):
    """float64 y = rmsnorm(KATA(q, k, v)) and its gradients."""
    leaves = [t.double().requires_grad_(True) for t in (q, k, v, w)]
    cl = c.double().requires_grad_(True) if c is not None else None
    o, _ = K.kata_fwd(*leaves[:3], M, None, variant, cl)
    y = X.rmsnorm(o, leaves[3], eps)
    gs = torch.autograd.grad((y * dy.double()).sum(), leaves + ([cl] if cl is not None else []))
    return y.detach(), gs


CASES = [  # B, T, HQ, H, M, variant, decay
    (1, 1, 1, 1, 4, "concat", False),
    (2, 200, 4, 4, 4, "concat", False),
    (1, 300, 4, 2, 2, "concat", False),   # GQA
    (1, 129, 2, 2, 1, "concat", False),
    (1, 200, 3, 3, 2, "sum", False),
    (1, 150, 2, 2, 4, "sum", False),
    (1, 257, 2, 2, 4, "concat", True),
]


@pytest.mark.parametrize("B,T,HQ,H,M,variant,decay", CASES,
                         ids=[f"{c[5]}{'_decay' if c[6] else ''}_M{c[4]}_T{c[1]}_HQ{c[2]}_H{c[3]}"
                              for c in CASES])
def test_onorm_fwd_bwd_parity(P, B, T, HQ, H, M, variant, decay):
    print(f"\nonorm {variant} decay={decay} B{B} T{T} HQ{HQ} H{H} M{M}", flush=True)
    q, k, v, dy, w, c = inputs(B, T, HQ, H, M, 7 * T + M, decay=decay)
    y_ref, g_ref = oracle(q, k, v, w, c, dy, M, variant)
    dev = [t.cuda().requires_grad_(True) for t in (q, k, v, w)]
    cd = c.cuda().requires_grad_(True) if c is not None else None
    y = P.parallel_kata_attn_onorm(*dev[:3], dev[3], 1e-5, M, None, variant, cd)
    assert y.dtype == torch.bfloat16 and y.shape == (B, T, HQ, 64)
    y.backward(dy.cuda())
    errs = {"y": mar(y, y_ref)}
    # dq, dk scale as |dO| |v| / |q| (o is invariant to the scale of q or k);
    # 10 % of that is the floor, with |dO| taken from dv = P^T dO
    m = lambda t: t.detach().abs().max().item()  # noqa: E731
    fl = {"dq": 0.1 * m(g_ref[2]) * m(v) / m(q), "dk": 0.1 * m(g_ref[2]) * m(v) / m(k)}
    for name, t, g in zip(("dq", "dk", "dv", "dw"), dev, g_ref):
        errs[name] = mar(t.grad, g, fl.get(name, 0.0))
    if cd is not None:
        errs["dc"] = mar(cd.grad, g_ref[4])
    print("  " + " ".join(f"{n} {e:.2e}" for n, e in errs.items()), flush=True)
    for n, e in errs.items():
        assert e < BAR[torch.bfloat16], (n, e)


def test_onorm_matches_unfused_chain(P):
    """Against the two-step HIP chain (KATA, then the RMSNorm kernels): o and
    den of the fused forward are the plain forward's bit for bit; y and the
    gradients differ only by the order of fp32 sums."""
    from linatt_amd.mixer import rms_norm
    q, k, v, dy, w, _ = inputs(2, 333, 4, 4, 4, 11)
    qd, kd, vd, wd = (t.cuda() for t in (q, k, v, w))
    o_plain, den_plain = P.parallel_kata_attn_fwd(qd, kd, vd, 4)
    # the fused forward's own o and den through the C ABI
    from linatt_amd import _lib
    L = _lib.load()
    o = torch.empty_like(o_plain)
    y = torch.empty_like(o_plain)
    den = torch.empty_like(den_plain)
    rstd = torch.empty_like(den_plain)
    _lib.check("linatt_kata_fwd_onorm", L.linatt_kata_fwd_onorm(
        _lib.ptr(qd), _lib.ptr(kd), _lib.ptr(vd), None, _lib.ptr(o), _lib.ptr(den), _lib.ptr(wd),
        1e-5, _lib.ptr(y), _lib.ptr(rstd), 2, 333, 4, 4, 64, 64, 4, 0.25, 0, _lib.LINATT_BFLOAT16,
        _lib.stream_of(qd)))
    torch.cuda.synchronize()
    assert torch.equal(o, o_plain) and torch.equal(den, den_plain)
    y_chain = rms_norm(o_plain, wd, 1e-5)
    assert mar(y, y_chain) < 8e-3  # one bf16 rounding apart at most

    leaves_f = [t.cuda().requires_grad_(True) for t in (q, k, v, w)]
    P.parallel_kata_attn_onorm(*leaves_f[:3], leaves_f[3], 1e-5, 4).backward(dy.cuda())
    leaves_u = [t.cuda().requires_grad_(True) for t in (q, k, v, w)]
    rms_norm(P.parallel_kata_attn(*leaves_u[:3], 4), leaves_u[3], 1e-5).backward(dy.cuda())
    for a, b, n in zip(leaves_f, leaves_u, ("dq", "dk", "dv", "dw")):
        e = mar(a.grad, b.grad)
        print(f"  fused vs chain {n} {e:.2e}", flush=True)
        assert e < 1e-2, (n, e)


def test_onorm_fp16_forward_and_no_weight(P):
    """fp16 runs fused without a gradient; no norm weight means weight 1."""
    q, k, v, _, w, _ = inputs(1, 190, 2, 2, 2, 23, dtype=torch.float16)
    y_ref, _ = oracle(q, k, v, torch.ones(64), None, torch.zeros(1, 190, 2, 64), 2, "concat")
    with torch.no_grad():
        y = P.parallel_kata_attn_onorm(q.cuda(), k.cuda(), v.cuda(), None, 1e-5, 2)
    assert y.dtype == torch.float16
    assert mar(y, y_ref) < BAR[torch.float16]


def test_onorm_repeat_runs_identical(P):
    q, k, v, dy, w, _ = inputs(2, 512, 4, 4, 4, 31)
    res = []
    for _ in range(2):
        leaves = [t.cuda().requires_grad_(True) for t in (q, k, v, w)]
        y = P.parallel_kata_attn_onorm(*leaves[:3], leaves[3], 1e-5, 4)
        y.backward(dy.cuda())
        res.append([y.detach()] + [t.grad for t in leaves])
    for a, b in zip(*res):
        assert torch.equal(a, b)
