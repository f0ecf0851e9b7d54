"""GPU parity of the SPD delta rule (``linatt_amd.flash_delta``, C ABI
``linatt_dkata_fwd``) against the float64 CPU oracle ``oracle.delta_kata``.

Inputs are drawn on the CPU from seeded generators, rounded once to the test
dtype, and the same rounded tensors feed both sides.  q and k are
l2-normalised per head, as the delta mixer does (``norm_q: l2``, ``norm_k:
l2`` in ``configs/model/kata_delta_m1_340m.yaml``), so that
``beta kappa(k, k) <= 1`` and the delta recursion stays bounded; beta is a
sigmoid of a normal draw.  Error metric: ``max|x - ref| / max|ref|`` per
tensor; bars: bfloat16 2e-2, float16 1e-2.
"""

import pytest
import torch

from oracle import delta_kata as DK

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 2e-2, torch.float16: 1e-2}


def mar(x, ref, floor=0.0):
    """max|x - ref| / max(max|ref|, floor).  The floor matters only where the
    exact gradient nearly vanishes: a normalised output at T = 1 is
    U_0 kappa / (kappa + eps), invariant to q and k up to eps, so dq and dk
    are ~eps-sized there and would be measured against their own rounding."""
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = max(ref.abs().max().item(), floor)
    return (x - ref).abs().max().item() / (den if den > 0 else 1.0)


def make(B, T, H, D, DV, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, D, generator=g), dim=-1).to(dtype)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, D, generator=g), dim=-1).to(dtype)
    v = torch.randn(B, T, H, DV, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    return q, k, v, beta


@pytest.fixture(scope="module")
def F():
    from linatt_amd import flash_delta as F
    return F


def dev(*ts):
    return [t.cuda() for t in ts]


SHAPES = [  # B, T, H
    (1, 1, 1),
    (2, 37, 2),
    (1, 64, 1),
    (1, 129, 3),
    (2, 300, 2),
    (1, 700, 2),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("scale", [None, 0.5, 1.0])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_forward_parity(F, shape, M, scale, dtype):
    B, T, H = shape
    q, k, v, beta = make(B, T, H, 64, 64, dtype, 7 + T + M)
    print(f"\nflash_delta B={B} T={T} H={H} M={M} scale={scale} {dtype}", flush=True)
    o_ref, U_ref, num_ref, den_ref = DK.flash_delta_fwd(q, k, v, beta, M, scale)
    qd, kd, vd, bd = dev(q, k, v, beta)
    tol = TOL[dtype]
    U = F.flash_delta_U(qd, kd, vd, bd, M, scale=scale)
    assert U.dtype == torch.float32 and U.shape == (B, T, H, 64)
    assert mar(U, U_ref) < tol, ("U", mar(U, U_ref))
    o = F.flash_delta(qd, kd, vd, bd, M, scale=scale)
    assert o.dtype == torch.float32
    assert mar(o, num_ref) < tol, ("num", mar(o, num_ref))
    on = F.flash_delta(qd, kd, vd, bd, M, scale=scale, normalize=True, eps=1e-5)
    on_ref = num_ref / (den_ref[..., None] + 1e-5)
    assert mar(on, on_ref) < tol, ("o normalised", mar(on, on_ref))
    den = F.flash_delta_den(qd, kd, M, scale=scale)
    assert mar(den, den_ref) < tol, ("den", mar(den, den_ref))
    num = F.flash_delta_readout(qd, kd, U, M, scale=scale)
    assert mar(num, num_ref) < tol, ("readout", mar(num, num_ref))


def test_config_full_size(F):
    """``kata_delta_m1_340m``: M = 1, H = 16 heads of 64, T = 2048,
    delta_scale 0.5, bf16 inputs (``kata/layer.py:409-418``)."""
    B, T, H, M = 1, 2048, 16, 1
    q, k, v, beta = make(B, T, H, 64, 64, torch.bfloat16, 11)
    beta = beta.bfloat16().float()  # the mixer hands beta over in bf16
    print(f"\nflash_delta config B={B} T={T} H={H} M={M}", flush=True)
    o_ref, U_ref, num_ref, den_ref = DK.flash_delta_fwd(q, k, v, beta, M, 0.5)
    qd, kd, vd, bd = dev(q, k, v, beta)
    o = F.flash_delta(qd, kd, vd, bd, M, scale=0.5)
    assert mar(o, num_ref) < 2e-2, mar(o, num_ref)
    U = F.flash_delta_U(qd, kd, vd, bd, M, scale=0.5)
    assert mar(U, U_ref) < 2e-2, mar(U, U_ref)


@pytest.mark.parametrize("M", [1, 2, 4])
def test_orthonormal_keys_overwrite(F, M):
    """Closed form, no oracle: with keys from the first E standard basis
    vectors (all in group 0), scale 1 and beta = 1, ``kappa(e_a, e_b) =
    [a == b]``, the rule overwrites, and a query ``e_a`` at time t reads the
    value last written under key a at or before t (zero if none).  (Basis
    vectors at the same position of different groups would collide: the
    sum-SPD score pairs every group of q with every group of k.)"""
    B, T, H, D = 1, 517, 2, 64
    nkeys = D // M
    g = torch.Generator().manual_seed(M)
    ki = torch.randint(0, nkeys, (B, T, H), generator=g)
    qi = torch.randint(0, nkeys, (B, T, H), generator=g)
    eye = torch.eye(D)
    k = eye[ki].bfloat16()
    q = eye[qi].bfloat16()
    v = torch.randn(B, T, H, D, generator=g).bfloat16()
    beta = torch.ones(B, T, H)
    want = torch.zeros(B, T, H, D)
    for b in range(B):
        for h in range(H):
            last = {}
            for t in range(T):
                last[int(ki[b, t, h])] = v[b, t, h].float()
                if int(qi[b, t, h]) in last:
                    want[b, t, h] = last[int(qi[b, t, h])]
    o = F.flash_delta(*dev(q, k, v, beta), M, scale=1.0)
    assert mar(o, want) < 1e-2, mar(o, want)


def test_causal_prefix_and_padding(F):
    """Rows t < T1 depend on tokens <= t only: a prefix run equals the prefix
    of a longer run, and zero padding (the mixer pads T up to a power of two,
    ``kata/layer.py:383-394``) changes nothing before it."""
    B, T, H, M = 2, 1500, 4, 2
    q, k, v, beta = dev(*make(B, T, H, 64, 64, torch.bfloat16, 3))
    full = F.flash_delta(q, k, v, beta, M, scale=0.5, normalize=True)
    T1 = 701
    pre = F.flash_delta(q[:, :T1], k[:, :T1], v[:, :T1], beta[:, :T1], M, scale=0.5,
                        normalize=True)
    # the two runs chunk the prefix identically, so only the readout's
    # key-tile schedule may differ: agreement to fp32 accumulation order
    assert mar(pre, full[:, :T1]) < 1e-5
    pad = 2048 - T
    zp = lambda x: torch.nn.functional.pad(x, (0, 0) * (x.dim() - 2) + (0, pad))  # noqa: E731
    padded = F.flash_delta(zp(q), zp(k), zp(v), zp(beta), M, scale=0.5, normalize=True)
    assert mar(padded[:, :T], full) < 1e-5


def test_deterministic(F):
    q, k, v, beta = dev(*make(2, 777, 3, 64, 64, torch.bfloat16, 5))
    a = F.flash_delta(q, k, v, beta, 4, scale=0.5)
    b = F.flash_delta(q, k, v, beta, 4, scale=0.5)
    assert torch.equal(a, b)


BWD_SHAPES = [(1, 1, 1), (2, 37, 2), (1, 129, 3), (2, 300, 2), (1, 700, 1)]


@pytest.mark.parametrize("shape", BWD_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("normalize", [False, True], ids=["raw", "norm"])
@pytest.mark.parametrize("scale,dtype", [(0.5, torch.bfloat16), (1.0, torch.bfloat16),
                                         (None, torch.bfloat16)], ids=["s0.5", "s1", "sE"])
def test_backward_parity(F, shape, M, normalize, scale, dtype):
    """dq, dk, dv, dbeta of <o, do> against float64 autograd through the
    oracle (the reference's _FlashDelta.backward differentiates the same
    function, kata/spd/flash_delta.py:1084-1108)."""
    B, T, H = shape
    q, k, v, beta = make(B, T, H, 64, 64, dtype, 31 + T + M)
    g = torch.Generator().manual_seed(5 + T)
    do = torch.randn(B, T, H, 64, generator=g)
    print(f"\nflash_delta bwd B={B} T={T} H={H} M={M} norm={normalize} scale={scale} {dtype}",
          flush=True)
    o_ref, dq_ref, dk_ref, dv_ref, db_ref = DK.flash_delta_fwd_bwd(q, k, v, beta, M, do, scale,
                                                                  normalize)
    qd, kd, vd, bd = (t.cuda().requires_grad_(True) for t in (q, k, v, beta))
    o = F.flash_delta(qd, kd, vd, bd, M, scale=scale, normalize=normalize)
    o.backward(do.cuda())
    tol = TOL[dtype]
    assert mar(o, o_ref) < tol, ("o", mar(o, o_ref))
    # 10% of the natural scale of dq, dk for a normalised output,
    # |do / (den + eps)| |v| / |q| (the output is a den-weighted average)
    m = lambda t: t.abs().max().item()  # noqa: E731
    if normalize:
        den = DK.flash_delta_fwd(q, k, v, beta, M, scale)[3]
        fl = 0.1 * m(do.double() / (den[..., None] + 1e-5)) * m(v.float()) / m(q.float())
    else:
        fl = 0.0
    for name, got, ref in (("dq", qd.grad, dq_ref), ("dk", kd.grad, dk_ref),
                           ("dv", vd.grad, dv_ref), ("dbeta", bd.grad, db_ref)):
        assert got.dtype == (torch.float32 if name == "dbeta" else dtype)
        e = mar(got, ref, fl if name in ("dq", "dk") else 0.0)
        assert e < tol, (name, e)


@pytest.mark.parametrize("T", [512, 513, 1025, 1600])
def test_super_chunk_boundaries(F, T):
    """The chunk-sequential passes run in super-chunks of 8 chunks (512
    tokens), with the other super-chunks' terms added by a parallel kernel:
    lengths at and just past those boundaries, forward and backward."""
    B, H, M = 1, 2, 2
    q, k, v, beta = make(B, T, H, 64, 64, torch.bfloat16, 40 + T)
    do = torch.randn(B, T, H, 64, generator=torch.Generator().manual_seed(T))
    print(f"\nflash_delta super-chunks T={T}", flush=True)
    o_ref, dq_ref, dk_ref, dv_ref, db_ref = DK.flash_delta_fwd_bwd(q, k, v, beta, M, do, 0.5)
    qd, kd, vd, bd = (t.cuda().requires_grad_(True) for t in (q, k, v, beta))
    o = F.flash_delta(qd, kd, vd, bd, M, scale=0.5)
    o.backward(do.cuda())
    for name, got, ref in (("o", o, o_ref), ("dq", qd.grad, dq_ref), ("dk", kd.grad, dk_ref),
                           ("dv", vd.grad, dv_ref), ("dbeta", bd.grad, db_ref)):
        e = mar(got, ref)
        assert e < 2e-2, (name, e)


def test_train_forward_keeps_no_U(F):
    """The training forward through the C ABI with U = NULL writes the same
    output, den and backward-visible workspace as with U given, and the
    backward (which never reads U) gives identical gradients either way."""
    from linatt_amd import _lib
    L = _lib.load()
    B, T, H, D, M = 1, 300, 2, 64, 2
    q, k, v, beta = dev(*make(B, T, H, D, D, torch.bfloat16, 77))
    do = torch.randn(B, T, H, D, device="cuda")
    dt = _lib.dtype_code(q.dtype)
    P, sp = _lib.ptr, _lib.stream_of(q)
    outs = []
    for with_u in (True, False):
        U = torch.empty(B, T, H, D, device="cuda") if with_u else None
        o = torch.empty(B, T, H, D, device="cuda")
        den = torch.empty(B, T, H, device="cuda")
        ws = torch.zeros(L.linatt_dkata_workspace_bytes(B, T, H, D, D, dt), device="cuda",
                         dtype=torch.uint8)
        _lib.check("linatt_dkata_fwd_train", L.linatt_dkata_fwd_train(
            P(q), P(k), P(v), P(beta), P(U), P(o), P(den), P(ws), B, T, H, D, D, M, 0.5, 0,
            1e-5, dt, sp))
        g = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
             torch.empty(B, T, H, device="cuda")]
        bws = torch.empty(L.linatt_dkata_bwd_workspace_bytes(B, T, H, D, D, dt), device="cuda",
                          dtype=torch.uint8)
        _lib.check("linatt_dkata_bwd", L.linatt_dkata_bwd(
            P(q), P(k), P(v), P(beta), P(U), None, P(den), P(do), *(P(t) for t in g), P(ws),
            P(bws), B, T, H, D, D, M, 0.5, 0, 1e-5, dt, sp))
        outs.append([o, den] + g)
        if with_u:
            ref = F.flash_delta_U(q, k, v, beta, M, scale=0.5)
            assert torch.equal(U, ref)
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("shape,M", [((2, 37, 2), 1), ((1, 300, 2), 4), ((1, 1, 1), 2)],
                         ids=["2x37x2_M1", "1x300x2_M4", "1x1x1_M2"])
def test_backward_fp16_runs_in_bf16(F, shape, M):
    """float16 inputs with a gradient run forward and backward in bfloat16:
    the output equals the bfloat16 op's on the converted inputs bit for bit,
    the gradients come back in float16 and meet the bfloat16 bar against the
    float64 oracle on the float16 inputs themselves."""
    B, T, H = shape
    q, k, v, beta = make(B, T, H, 64, 64, torch.float16, 90 + T)
    do = torch.randn(B, T, H, 64, generator=torch.Generator().manual_seed(91 + T))
    o_ref, dq_ref, dk_ref, dv_ref, db_ref = DK.flash_delta_fwd_bwd(q, k, v, beta, M, do, None, False)
    qd, kd, vd, bd = (t.cuda().requires_grad_(True) for t in (q, k, v, beta))
    o = F.flash_delta(qd, kd, vd, bd, M)
    o.backward(do.cuda())
    with torch.no_grad():
        o_bf = F.flash_delta(*(t.cuda().bfloat16() for t in (q, k, v)), beta.cuda(), M)
    assert torch.equal(o, o_bf)
    bar = TOL[torch.bfloat16]
    assert mar(o, o_ref) < bar
    for name, got, ref in (("dq", qd.grad, dq_ref), ("dk", kd.grad, dk_ref),
                           ("dv", vd.grad, dv_ref), ("dbeta", bd.grad, db_ref)):
        assert got.dtype == (torch.float32 if name == "dbeta" else torch.float16), name
        e = mar(got, ref)
        print(f"  fp16-in {name} {e:.2e}", flush=True)
        assert e < bar, (name, e)


def test_backward_fp32_raises(F):
    q, k, v, beta = make(1, 64, 1, 64, 64, torch.float32, 1)
    qd = q.cuda().requires_grad_(True)
    with pytest.raises(NotImplementedError, match="bfloat16"):
        F.flash_delta(qd, k.cuda(), v.cuda(), beta.cuda(), 1)


def test_backward_config_full_size(F):
    """The kata_delta_m1_340m shape (H=16, T=2048, M=1, scale 0.5), three heads
    against the oracle."""
    B, T, H, M = 1, 2048, 16, 1
    q, k, v, beta = make(B, T, H, 64, 64, torch.bfloat16, 13)
    do = torch.randn(B, T, H, 64, generator=torch.Generator().manual_seed(14))
    qd, kd, vd, bd = (t.cuda().requires_grad_(True) for t in (q, k, v, beta))
    F.flash_delta(qd, kd, vd, bd, M, scale=0.5).backward(do.cuda())
    for h in (0, 7, 15):
        sl = lambda x: x[:, :, h:h + 1]  # noqa: E731
        _, dq_ref, dk_ref, dv_ref, db_ref = DK.flash_delta_fwd_bwd(
            sl(q), sl(k), sl(v), sl(beta), M, sl(do), 0.5)
        for name, got, ref in (("dq", qd.grad, dq_ref), ("dk", kd.grad, dk_ref),
                               ("dv", vd.grad, dv_ref), ("dbeta", bd.grad, db_ref)):
            e = mar(sl(got), ref)
            assert e < 2e-2, (name, h, e)


def test_backward_deterministic(F):
    q, k, v, beta = make(2, 500, 3, 64, 64, torch.bfloat16, 8)
    do = torch.randn(2, 500, 3, 64, generator=torch.Generator().manual_seed(9)).cuda()
    res = []
    for _ in range(2):
        qd, kd, vd, bd = (t.cuda().requires_grad_(True) for t in (q, k, v, beta))
        F.flash_delta(qd, kd, vd, bd, 2, scale=0.5, normalize=True).backward(do)
        res.append([t.grad.clone() for t in (qd, kd, vd, bd)])
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_unsupported_shape_raises(F):
    q, k, v, beta = dev(*make(1, 8, 1, 64, 32, torch.bfloat16, 1))
    with pytest.raises(NotImplementedError, match="no kernel"):
        F.flash_delta(q, k, v, beta, 1)
    q32, k32, v32 = (x.float() for x in dev(*make(1, 8, 1, 64, 64, torch.bfloat16, 1)[:3]))
    with pytest.raises((NotImplementedError, TypeError)):
        F.flash_delta(q32, k32, v32, beta, 1)


@pytest.mark.parametrize("M", [1, 2, 4])
def test_readout_keeps_float32_accumulator(F, M):
    """The readout as the reference's kernel computes it
    (``kata/spd/flash_delta.py:915-972``): A_qk and U rounded to bf16, the
    products summed in float32 and stored unrounded.  Against that
    computation in float64 (same roundings), the HIP readout is within
    1e-3 (measured at most 3.5e-4): only the fp32 sum order and an
    occasional one-ulp difference in a rounded A_qk element remain (no
    16-bit rounding of the result)."""
    B, T, H = 2, 300, 2
    q, k, v, beta = make(B, T, H, 64, 64, torch.bfloat16, 40 + M)
    qd, kd, vd, bd = dev(q, k, v, beta)
    U = F.flash_delta_U(qd, kd, vd, bd, M, scale=0.5)
    num = F.flash_delta_readout(qd, kd, U, M, scale=0.5)
    A = torch.tril(DK.kappa_gram(q.double(), k.double(), M, 0.5))      # (B, H, T, T)
    A16 = A.float().bfloat16().double()
    U16 = U.cpu().bfloat16().double().transpose(1, 2)                  # (B, H, T, DV)
    ref = (A16 @ U16).transpose(1, 2)
    e = mar(num, ref)
    print(f"\nreadout M={M}: {e:.2e} against the reference's roundings", flush=True)
    assert e < 1e-3
    # the training forward's output is that readout of its own U: num itself
    o = F.flash_delta(qd, kd, vd, bd, M, scale=0.5)
    assert mar(o, num) < 2e-3
