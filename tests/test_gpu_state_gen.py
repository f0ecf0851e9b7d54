"""GPU parity of the state form of every flash score (the decode cache,
``linatt_amd.kata_cache.parallel_kata_attn_cached`` over
``linatt_kata_gen_decode`` / ``_readout`` / ``_update``) against the float64
oracle's parallel form.

A sequence is fed as a prefill, single-token decode steps, a prefill
continued from the state, and more decode steps; the outputs, concatenated,
must equal ``oracle.kata.kata_fwd`` over the whole sequence (the flash
forward the reference runs without a cache) within the bf16 bar of 2e-2.
Covered: the concat score with one group (P = 4096 state rows), the sum
score (M = 2, 4), the decayed concat score (each call gets its own
cumulative log-decay, as the mixer computes it), and the offset gate's
padded width (dk = 128, two groups of 64 with zero padding, decayed, the
``kataconv_cat_l2_gdn_340m`` mixer).  The cache keeps a new state packed
(rows a <= b of each group); the same calls continued from the unpacked
state must keep the full layout's rows a <= b equal to the packed rows bit
for bit, and agree on the outputs within rounding.
"""

import math

import pytest
import torch

from oracle import kata as K

pytestmark = pytest.mark.gpu
BAR = 2e-2


def mar(x, ref):
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return (x - ref).abs().max().item() / ref.abs().max().item()


def gen(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * std


CASES = {  # name: (dk, M, variant, decay, padded)
    "concat_M1": (64, 1, "concat", False, False),
    "sum_M2": (64, 2, "sum", False, False),
    "sum_M4": (64, 4, "sum", False, False),
    "concat_M2_decay": (64, 2, "concat", True, False),
    "offset_gate_dk128_decay": (128, 2, "concat", True, True),
}
# calls: prefill, 4 decode steps, a continued prefill, 3 decode steps
SPLITS = [0, 150, 151, 152, 153, 154, 224, 225, 226, 227]


@pytest.mark.parametrize("case", list(CASES))
def test_state_form_equals_parallel(case):
    from linatt_amd.kata_cache import parallel_kata_attn_cached
    dk, M, variant, decay, padded = CASES[case]
    B, H, T, dv = 2, 3, SPLITS[-1], 64
    print(f"\nstate form {case}: B{B} H{H} T{T} dk{dk} M{M}", flush=True)
    seed = 5 + dk + M
    q, k = gen((B, T, H, dk), seed, 0.5), gen((B, T, H, dk), seed + 1, 0.5)
    if padded:  # each group: 32 live dims, the gate coordinate, zero padding
        gate = torch.sigmoid(gen((B, T, H), seed + 2))
        for g in range(M):
            q[..., 64 * g + 33:64 * (g + 1)] = 0
            k[..., 64 * g + 33:64 * (g + 1)] = 0
            q[..., 64 * g + 32] = gate
            k[..., 64 * g + 32] = 1.0
    v = gen((B, T, H, dv), seed + 3)
    q, k, v = (t.bfloat16() for t in (q, k, v))
    scale = (1.0 / 32) ** 0.5 if padded else None
    c = None
    if decay:
        c = -(gen((B, T, H), seed + 4).abs() * 0.05).cumsum(1)
    o_ref, _ = K.kata_fwd(q.double(), k.double(), v.double(), M, scale, variant,
                          c.double() if c is not None else None)

    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    state, outs = None, []
    for s, e in zip(SPLITS[:-1], SPLITS[1:]):
        cc = None
        if decay:  # the call's own cumulative log-decay, from the stored state at 0
            cc = (c[:, s:e] - (c[:, s - 1:s] if s > 0 else 0.0)).cuda()
        o, state = parallel_kata_attn_cached(qd[:, s:e], kd[:, s:e], vd[:, s:e], state, M, scale,
                                             variant=variant, c=cc)
        assert o.shape == (B, e - s, H, dv) and o.dtype == torch.bfloat16
        outs.append(o)
    o_inc = torch.cat(outs, dim=1)
    assert state.offset == T and state.variant == variant
    errs = [mar(o_inc[:, s:e], o_ref[:, s:e]) for s, e in zip(SPLITS[:-1], SPLITS[1:])]
    print("  per call: " + " ".join(f"{x:.1e}" for x in errs), flush=True)
    assert max(errs) < BAR


def test_state_form_repeat_runs_identical():
    from linatt_amd.kata_cache import parallel_kata_attn_cached
    q, k, v = (gen((1, 100, 2, 64), 50 + i, 0.5).bfloat16().cuda() for i in range(3))
    res = []
    for _ in range(2):
        o1, st = parallel_kata_attn_cached(q[:, :90], k[:, :90], v[:, :90], None, 2, variant="sum")
        o2, st = parallel_kata_attn_cached(q[:, 90:91], k[:, 90:91], v[:, 90:91], st, 2,
                                           variant="sum")
        res.append((o1, o2, st.S.clone(), st.z.clone()))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_state_form_rejects_mismatched_state():
    from linatt_amd.kata_cache import parallel_kata_attn_cached
    q = gen((1, 8, 2, 64), 60).bfloat16().cuda()
    _, st = parallel_kata_attn_cached(q, q, q, None, 2, None, variant="sum")
    with pytest.raises(ValueError, match="state is for the sum score"):
        parallel_kata_attn_cached(q, q, q, st, 2, None, variant="concat")


def _inputs(case, B, H, T):
    dk, M, variant, decay, padded = CASES[case]
    seed = 7 + dk + M
    q, k = gen((B, T, H, dk), seed, 0.5), gen((B, T, H, dk), seed + 1, 0.5)
    v = gen((B, T, H, 64), seed + 3)
    c = -(gen((B, T, H), seed + 4).abs() * 0.05).cumsum(1) if decay else None
    scale = (1.0 / 32) ** 0.5 if padded else None
    return q.bfloat16().cuda(), k.bfloat16().cuda(), v.bfloat16().cuda(), c, scale


@pytest.mark.parametrize("case", list(CASES))
def test_packed_state_equals_full(case):
    from linatt_amd import _lib, spd_state
    from linatt_amd.kata_cache import KataState, parallel_kata_attn_cached, state_rows
    dk, M, variant, decay, padded = CASES[case]
    G = 1 if variant == "sum" else M
    B, H, T = 2, 3, 160
    splits = [0, 100, 101, 102, 140, 141, 160]
    print(f"\npacked vs full state {case}: B{B} H{H} T{T}", flush=True)
    q, k, v, c, scale = _inputs(case, B, H, T)
    Pf, Pp = state_rows(dk, M, variant), state_rows(dk, M, variant, True)
    L = _lib.load()
    var = 1 if variant == "sum" else 0
    sc = scale if scale is not None else 1.0 / math.sqrt(dk // M)  # the cache's default

    def cc(s, e):
        if c is None:
            return None
        return (c[:, s:e] - (c[:, s - 1:s] if s > 0 else 0.0)).cuda()

    # a state from zero through the C-ABI in both layouts
    n0 = splits[1]
    c0 = cc(0, n0)
    c0 = c0.contiguous() if c0 is not None else None
    kk, vv = k[:, :n0].contiguous(), v[:, :n0].contiguous()
    full = (torch.empty(B, H, Pf, 64, device="cuda"), torch.empty(B, H, Pf, device="cuda"))
    pack = (torch.empty(B, H, Pp, 64, device="cuda"), torch.empty(B, H, Pp, device="cuda"))
    for (S, z), vr in ((full, var), (pack, var | _lib.LINATT_KATA_PACKED_STATE)):
        _lib.check("linatt_kata_gen_update", L.linatt_kata_gen_update(
            _lib.ptr(kk), _lib.ptr(vv), _lib.ptr(c0), _lib.ptr(S), _lib.ptr(z), 0, B, n0, H, dk, 64,
            M, vr, float(sc), _lib.dtype_code(v.dtype), _lib.stream_of(v)))
    Sp, zp = spd_state.pack_state(*full, G)
    assert torch.equal(Sp, pack[0]) and torch.equal(zp, pack[1])

    # the cache from here on: the packed state and its unpacked copy
    o_p, st_p = parallel_kata_attn_cached(q[:, :n0], k[:, :n0], v[:, :n0], None, M, scale,
                                          variant=variant, c=cc(0, n0))
    assert st_p.S.shape == (B, H, Pp, 64) and st_p.z.shape == (B, H, Pp)
    assert torch.equal(st_p.S, pack[0]) and torch.equal(st_p.z, pack[1])
    st_f = KataState(*spd_state.unpack_state(st_p.S, st_p.z, G), n0, variant, M)
    assert torch.equal(st_f.S, full[0]) and torch.equal(st_f.z, full[1])
    for s, e in zip(splits[1:-1], splits[2:]):
        o_p, st_p = parallel_kata_attn_cached(q[:, s:e], k[:, s:e], v[:, s:e], st_p, M, scale,
                                              variant=variant, c=cc(s, e))
        o_f, st_f = parallel_kata_attn_cached(q[:, s:e], k[:, s:e], v[:, s:e], st_f, M, scale,
                                              variant=variant, c=cc(s, e))
        assert st_f.S.shape[2] == Pf and st_p.S.shape[2] == Pp
        Sp, zp = spd_state.pack_state(st_f.S, st_f.z, G)
        assert torch.equal(Sp, st_p.S) and torch.equal(zp, st_p.z), (s, e)
        err = mar(o_p, o_f)
        print(f"  call {s}:{e} packed vs full o {err:.1e}", flush=True)
        assert err < 1e-2


DIRECT = [  # (dk, M, variant, packed, decay, dtype): group widths 128 (M = 1), 64, 32 and 16
    (128, 1, "concat", False, False, torch.bfloat16),
    (128, 1, "concat", True, True, torch.bfloat16),
    (64, 2, "concat", True, False, torch.bfloat16),
    (64, 2, "sum", False, True, torch.bfloat16),
    (64, 4, "sum", True, False, torch.bfloat16),
    (128, 4, "concat", True, False, torch.bfloat16),
    (64, 2, "concat", True, True, torch.float16),
    (64, 2, "concat", True, True, torch.float32),
    (64, 4, "sum", False, False, torch.float32),
    (48, 3, "sum", True, False, torch.bfloat16),  # three groups: a group count known at run time
    (128, 8, "sum", False, False, torch.bfloat16),
]
# long prompts: the bf16 products accumulate over thousands of tokens
DIRECT_LONG = [(64, 1, "concat", True, True, torch.bfloat16, 2048),
               (64, 4, "sum", True, False, torch.bfloat16, 1536)]
DIRECT_BAR = {torch.bfloat16: 2e-2, torch.float16: 1e-2, torch.float32: 1e-4}


@pytest.mark.parametrize("dk,M,variant,packed,decay,dtype,T",
                         [c + (150,) for c in DIRECT] + DIRECT_LONG)
def test_update_readout_direct(dk, M, variant, packed, decay, dtype, T):
    """``linatt_kata_gen_update`` from zero then ``linatt_kata_gen_readout``
    through the C ABI against the state formulas in float64 with the full
    feature map psi(x) = vec(scale x_g x_g^T) (summed over g for the sum
    score), including group widths the cached attention cannot reach.  16-bit
    inputs run the matrix-core kernels (bf16 products), float32 inputs the
    float32 ones (held to 1e-4)."""
    from linatt_amd import _lib, spd_state
    from linatt_amd.kata_cache import state_rows
    B, H, dv = 2, 3, 64
    E = dk // M
    G = 1 if variant == "sum" else M
    print(f"\ndirect gen update/readout dk{dk} M{M} {variant} packed={packed} decay={decay} "
          f"{dtype} T{T}", flush=True)
    g0 = 900 + dk + M + 7 * packed
    q, k = gen((B, T, H, dk), g0, 0.5).to(dtype), gen((B, T, H, dk), g0 + 1, 0.5).to(dtype)
    v = gen((B, T, H, dv), g0 + 2).to(dtype)
    c = -(gen((B, T, H), g0 + 3).abs() * 0.05).cumsum(1) if decay else None
    o_in = gen((B, T, H, dv), g0 + 4).to(dtype)
    den_in = gen((B, T, H), g0 + 5).abs() + 0.5
    scale = 1.0 / math.sqrt(E)

    def psi(x):
        xg = x.double().reshape(*x.shape[:-1], M, E)
        outer = scale * xg[..., :, None] * xg[..., None, :]
        if variant == "sum":
            return outer.sum(-3).flatten(-2)
        return outer.flatten(-3)

    pk, pq = psi(k), psi(q)  # (B, T, H, Pf)
    wk = torch.ones(B, T, H, dtype=torch.float64)
    fq = torch.ones(B, T, H, dtype=torch.float64)
    if decay:
        cd = c.double()
        wk = torch.exp(cd[:, -1:] - cd)
        fq = torch.exp(cd)
    S_ref = torch.einsum("bthp,bthn->bhpn", pk * wk[..., None], v.double())
    z_ref = (pk * wk[..., None]).sum(1)
    num = o_in.double() * den_in.double()[..., None] + fq[..., None] * torch.einsum(
        "bthp,bhpn->bthn", pq, S_ref)
    den = den_in.double() + fq * torch.einsum("bthp,bhp->bth", pq, z_ref)
    o_ref = num / den.clamp_min(1e-6)[..., None]

    L = _lib.load()
    var = (1 if variant == "sum" else 0) | (_lib.LINATT_KATA_PACKED_STATE if packed else 0)
    P = state_rows(dk, M, variant, packed)
    assert L.linatt_kata_gen_state_rows(dk, M, var) == P
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    cdv = c.float().cuda() if decay else None
    S = torch.empty(B, H, P, dv, device="cuda")
    z = torch.empty(B, H, P, device="cuda")
    code, sp = _lib.dtype_code(v.dtype), _lib.stream_of(vd)
    _lib.check("linatt_kata_gen_update", L.linatt_kata_gen_update(
        _lib.ptr(kd), _lib.ptr(vd), _lib.ptr(cdv), _lib.ptr(S), _lib.ptr(z), 0, B, T, H, dk, dv,
        M, var, scale, code, sp))
    o = o_in.cuda()
    dn = den_in.float().cuda()
    _lib.check("linatt_kata_gen_readout", L.linatt_kata_gen_readout(
        _lib.ptr(qd), _lib.ptr(cdv), _lib.ptr(S), _lib.ptr(z), _lib.ptr(o), _lib.ptr(dn), B, T, H,
        dk, dv, M, var, scale, 1e-6, code, sp))
    torch.cuda.synchronize()
    S_c, z_c = S.cpu(), z.cpu()
    if packed:
        S_c, z_c = spd_state.unpack_state(S_c, z_c, G)
    errs = (mar(S_c, S_ref), mar(z_c, z_ref), mar(o, o_ref), mar(dn, den.clamp_min(1e-6)))
    print("  S %.1e z %.1e o %.1e den %.1e" % errs, flush=True)
    assert max(errs) < DIRECT_BAR[dtype]


@pytest.mark.parametrize("variant,M,dtype", [("sum", 2, torch.bfloat16), ("concat", 1, torch.float16),
                                             ("concat", 4, torch.float16)])
def test_single_token_prompt_then_decode(variant, M, dtype):
    """A one-token prompt into an empty cache (the state update over T = 1),
    then decode steps and a short continued prefill, against the oracle's
    parallel form; fp16 inputs run the bf16 matrix-core products."""
    from linatt_amd.kata_cache import parallel_kata_attn_cached
    B, H, dk = 2, 3, 64
    splits = [0, 1, 2, 3, 40, 41]
    T = splits[-1]
    print(f"\nsingle-token prompt: {variant} M{M} {dtype}", flush=True)
    q, k = gen((B, T, H, dk), 80 + M, 0.5).to(dtype), gen((B, T, H, dk), 81 + M, 0.5).to(dtype)
    v = gen((B, T, H, 64), 82 + M).to(dtype)
    o_ref, _ = K.kata_fwd(q.double(), k.double(), v.double(), M, None, variant, None)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    st, outs = None, []
    for s, e in zip(splits[:-1], splits[1:]):
        o, st = parallel_kata_attn_cached(qd[:, s:e], kd[:, s:e], vd[:, s:e], st, M, variant=variant)
        assert o.dtype == dtype and o.shape == (B, e - s, H, 64)
        outs.append(o)
    err = mar(torch.cat(outs, 1), o_ref)
    print(f"  max rel err {err:.1e}", flush=True)
    assert err < (1e-2 if dtype == torch.float16 else BAR)


@pytest.mark.parametrize("dk,M,variant,packed,decay", [(64, 1, "concat", True, False),
                                                       (64, 2, "sum", True, True),
                                                       (128, 2, "concat", False, True),
                                                       (64, 2, "sum", False, False)])
def test_split_decode_equals_decode(dk, M, variant, packed, decay):
    """``linatt_kata_gen_decode_split`` (each (b, h)'s rows over several
    workgroups, partials added in a second launch) against
    ``linatt_kata_gen_decode``: the updated S and z bit for bit (each row is
    updated the same way), o to fp32 rounding of the final sums."""
    from linatt_amd import _lib
    from linatt_amd.kata_cache import state_rows
    B, H = 2, 5
    E = dk // M
    print(f"\nsplit decode dk{dk} M{M} {variant} packed={packed} decay={decay}", flush=True)
    L = _lib.load()
    var = (1 if variant == "sum" else 0) | (_lib.LINATT_KATA_PACKED_STATE if packed else 0)
    P = state_rows(dk, M, variant, packed)
    nws = L.linatt_kata_gen_decode_workspace_bytes(B, H, dk, M, var)
    assert nws > 0  # ten (b, h) pairs: the step splits
    S0 = (gen((B, H, P, 64), 500 + dk + M) * 0.05).cuda()
    z0 = (gen((B, H, P), 501 + dk + M).abs() + 0.5).cuda()
    q, k, v = (gen((B, H, w), 502 + i, 0.5).bfloat16().cuda() for i, w in enumerate((dk, dk, 64)))
    c = torch.full((B, H), -0.02, device="cuda") if decay else None
    outs = []
    for split in (False, True):
        S, z = S0.clone(), z0.clone()
        o = torch.empty(B, H, 64, device="cuda", dtype=torch.bfloat16)
        args = (_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(c), _lib.ptr(S), _lib.ptr(z), _lib.ptr(o))
        tail = (B, H, dk, 64, M, var, 1.0 / math.sqrt(E), 1e-6, 1, _lib.stream_of(q))
        if split:
            ws = torch.empty(nws, device="cuda", dtype=torch.uint8)
            _lib.check("split", L.linatt_kata_gen_decode_split(*args, _lib.ptr(ws), nws, *tail))
        else:
            _lib.check("decode", L.linatt_kata_gen_decode(*args, *tail))
        outs.append((S, z, o))
    torch.cuda.synchronize()
    (S1, z1, o1), (S2, z2, o2) = outs
    assert torch.equal(S1, S2) and torch.equal(z1, z2)
    err = mar(o2, o1)
    print(f"  o split vs one workgroup {err:.1e}", flush=True)
    assert err < 1e-2
