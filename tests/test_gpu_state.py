"""GPU parity of the psi-state KATA prefill and decode step
against the float64 CPU oracle (``oracle/kata.py``: ``kata_prefill_fwd_state_form``,
``kata_state_prefill``, ``kata_decode_step``, ``kata_fwd``, themselves pinned by
``tests/test_oracle_kata.py::test_state_form``).

Inputs are seeded on the CPU, rounded once to bf16, and the same rounded
tensors (upcast) feed the oracle.  Metric: max-abs-relative error per
tensor, bar 2e-2 (bf16).  Every case calls the C ABI through
``linatt_amd.spd_state``.
"""

import math

import pytest
import torch

from oracle import kata as K

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
TOL = 2e-2


def mar(x, ref):
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = ref.abs().max().item()
    return (x - ref).abs().max().item() / (den if den > 0 else 1.0)


def gen(shape, seed, std=0.125):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(BF)


@pytest.fixture(scope="module")
def S_():
    from linatt_amd import spd_state as S_
    return S_


@pytest.mark.parametrize("M", [4, 2])
@pytest.mark.parametrize("case", [(1, 1, 1, 128), (2, 300, 2, 128), (1, 1000, 3, 256),
                                  (1, 640, 2, 128), (2, 257, 1, 1024), (1, 800, 4, 512),
                                  (2, 1000, 4, 256)],
                         ids=lambda c: "B{}T{}H{}L{}".format(*c))
def test_prefill_parity(S_, M, case):
    B, T, H, Lseg = case
    print(f"case {case} M={M}", flush=True)
    q, k, v = gen((B, T, H, 64), 1 + T), gen((B, T, H, 64), 2 + T), gen((B, T, H, 64), 3 + T)
    o_ref, den_ref, S_ref, z_ref = K.kata_prefill_fwd_state_form(q, k, v, M, eps=1e-6)
    dev = torch.device("cuda")
    o, den, S, z = S_.kata_prefill(q.to(dev), k.to(dev), v.to(dev), num_groups=M, seg_len=Lseg)
    assert o.dtype == BF and den.dtype == torch.float32
    for name, x, ref in (("o", o, o_ref), ("den", den, den_ref), ("S", S, S_ref), ("z", z, z_ref)):
        e = mar(x, ref)
        assert e < TOL, (name, e)


@pytest.mark.parametrize("M", [4, 2])
def test_prefill_den_nonzero_mean_keys(S_, M):
    """Keys and queries with a non-zero mean and unequal per-dimension
    scales: every psi-feature sum z grows with the prefix, the case where a
    single 16-bit rounding of z would cost den its accuracy (about 4e-4
    relative here, computed on the CPU; hi + lo parts give about 2e-5), so
    den is checked to 1e-4."""
    B, T, H = 1, 3000, 2
    g = torch.Generator().manual_seed(77)
    scale_d = torch.linspace(0.05, 0.3, 64)
    mk = lambda: (torch.randn(B, T, H, 64, generator=g) * scale_d + 0.2).to(BF)  # noqa: E731
    q, k, v = mk(), mk(), gen((B, T, H, 64), 78)
    o_ref, den_ref, S_ref, z_ref = K.kata_prefill_fwd_state_form(q, k, v, M, eps=1e-6)
    dev = torch.device("cuda")
    o, den, S, z = S_.kata_prefill(q.to(dev), k.to(dev), v.to(dev), num_groups=M, seg_len=256)
    errs = {n: mar(x, r) for n, x, r in (("o", o, o_ref), ("den", den, den_ref), ("z", z, z_ref))}
    print(errs, flush=True)
    assert errs["o"] < TOL and errs["z"] < 1e-5
    assert errs["den"] < 1e-4, errs


def test_head_major_scan_cat(S_):
    """Reference layout (B, H, T, D) through spd_chunk_scan_cat."""
    B, T, H = 1, 700, 2
    q, k, v = gen((B, T, H, 64), 11), gen((B, T, H, 64), 12), gen((B, T, H, 64), 13)
    o_ref, den_ref, _, _ = K.kata_prefill_fwd_state_form(q, k, v, 4, eps=1e-6)
    dev = torch.device("cuda")
    hm = lambda x: x.transpose(1, 2).contiguous().to(dev)  # noqa: E731
    o, den = S_.spd_chunk_scan_cat(hm(q), hm(k), hm(v), 4)
    assert o.shape == (B, H, T, 64) and den.shape == (B, H, T)
    assert mar(o.transpose(1, 2), o_ref) < TOL
    assert mar(den.transpose(1, 2), den_ref) < TOL


@pytest.mark.parametrize("T", [1, 37, 64, 129, 700])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_scan_cat_linear_feature(S_, T, dtype):
    """spd_chunk_scan_cat(feature="linear") (linatt_linear_scan_fwd) against the
    float64 dense causal form.  q and k have a positive mean so that every
    den stays far above the eps clamp: near a zero den the output amplifies
    rounding without bound, in the reference too."""
    B, H, M = 2, 3, 4
    g = torch.Generator().manual_seed(T)
    q = (torch.randn(B, T, H, 64, generator=g) * 0.125 + 0.1).to(dtype)
    k = (torch.randn(B, T, H, 64, generator=g) * 0.125 + 0.1).to(dtype)
    v = torch.randn(B, T, H, 64, generator=g).to(dtype)
    print(f"\nlinear scan T={T} {dtype}", flush=True)
    o_ref, den_ref = K.linear_attn_dense(q, k, v, 1 / math.sqrt(64 // M))
    dev = torch.device("cuda")
    hm = lambda x: x.transpose(1, 2).contiguous().to(dev)  # noqa: E731
    o, den = S_.spd_chunk_scan_cat(hm(q), hm(k), hm(v), M, feature="linear")
    assert o.dtype == dtype and o.shape == (B, H, T, 64) and den.shape == (B, H, T)
    tol = TOL if dtype == BF else 1e-2
    assert mar(o.transpose(1, 2), o_ref) < tol, mar(o.transpose(1, 2), o_ref)
    assert mar(den.transpose(1, 2), den_ref) < 1e-3, mar(den.transpose(1, 2), den_ref)


def test_scan_cat_linear_clamp(S_):
    """Every q.k negative: den is the eps floor and o = num / eps (bf16: the
    outputs reach ~1e5, past fp16's range)."""
    B, T, H = 1, 150, 2
    g = torch.Generator().manual_seed(5)
    q = (-0.1 * (1 + 0.1 * torch.rand(B, T, H, 64, generator=g))).to(BF)
    k = (0.1 * (1 + 0.1 * torch.rand(B, T, H, 64, generator=g))).to(BF)
    v = torch.randn(B, T, H, 64, generator=g).to(BF)
    eps = 1e-4
    o_ref, den_ref = K.linear_attn_dense(q, k, v, 0.25, eps)
    assert (den_ref == eps).all()
    dev = torch.device("cuda")
    hm = lambda x: x.transpose(1, 2).contiguous().to(dev)  # noqa: E731
    o, den = S_.spd_chunk_scan_cat(hm(q), hm(k), hm(v), 4, eps=eps, feature="linear")
    assert (den == eps).all()
    assert mar(o.transpose(1, 2), o_ref) < TOL


@pytest.mark.parametrize("M", [4, 2])
def test_decode_equals_parallel_row(S_, M):
    """Decode after an n-token prefill == row n of the dense parallel form."""
    B, n, H = 2, 333, 3
    q, k, v = gen((B, n + 1, H, 64), 21), gen((B, n + 1, H, 64), 22), gen((B, n + 1, H, 64), 23)
    dev = torch.device("cuda")
    _, _, S, z = S_.kata_prefill(q[:, :n].to(dev), k[:, :n].to(dev), v[:, :n].to(dev),
                                 num_groups=M, seg_len=128)
    S0, z0 = S.cpu().double(), z.cpu().double()
    o = S_.kata_decode_step(S, z, q[:, n].to(dev), k[:, n].to(dev), v[:, n].to(dev), num_groups=M)
    o_par, _ = K.kata_fwd(q, k, v, M)
    assert mar(o, o_par[:, n]) < TOL
    o_ref, S_ref, z_ref = K.kata_decode_step(S0, z0, q[:, n], k[:, n], v[:, n], M)
    assert mar(o, o_ref) < TOL
    assert mar(S, S_ref) < TOL
    assert mar(z, z_ref) < TOL


def test_decode_multi_step(S_):
    """Eight decode steps at batch 4 from a zero state match the oracle step by step."""
    B, H, M = 4, 2, 4
    P = M * 16 * 16
    dev = torch.device("cuda")
    S = torch.zeros(B, H, P, 64, device=dev)
    z = torch.zeros(B, H, P, device=dev)
    Sr = torch.zeros(B, H, P, 64, dtype=torch.float64)
    zr = torch.zeros(B, H, P, dtype=torch.float64)
    for i in range(8):
        q, k, v = gen((B, H, 64), 100 + i), gen((B, H, 64), 200 + i), gen((B, H, 64), 300 + i)
        o = S_.kata_decode_step(S, z, q.to(dev), k.to(dev), v.to(dev), num_groups=M)
        o_ref, Sr, zr = K.kata_decode_step(Sr, zr, q, k, v, M)
        assert mar(o, o_ref) < TOL, i
    assert mar(S, Sr) < TOL and mar(z, zr) < TOL


def _row_ref(q, k, v, b, h, t, M, eps=1e-6):
    """Row t of the causal output in float64 (O(t) work)."""
    E = 64 // M
    scale = 1.0 / math.sqrt(E)
    qt = q[b, t, h].double().reshape(M, E)
    ks = k[b, :t + 1, h].double().reshape(t + 1, M, E)
    A = ((ks * qt).sum(-1) * scale).pow(2).sum(-1)  # (t+1,)
    den = max(A.sum().item(), eps)
    return (A[:, None] * v[b, :t + 1, h].double()).sum(0) / den, den


def test_config5_full_size(S_):
    """B=1 H=12 D=64 M=4 bf16, T=32768 prefill (seed 4)
    -> fp32 state, then decode steps at batch 64 (prefill state broadcast,
    fresh q, k, v ~ N(0,1)/8 from seed 4000+i).  Sampled output rows and
    state rows are checked against float64 sums over the whole prefix; the
    decode steps against the float64 decode step on two (b, h) slices."""
    B, T, H, M = 1, 32768, 12, 4
    g = torch.Generator().manual_seed(4)
    q, k, v = ((torch.randn(B, T, H, 64, generator=g) / 8).to(BF) for _ in range(3))
    dev = torch.device("cuda")
    o, den, S, z = S_.kata_prefill(q.to(dev), k.to(dev), v.to(dev), num_groups=M)
    assert torch.isfinite(o.float()).all() and torch.isfinite(S).all()
    oc, denc = o.cpu(), den.cpu()
    for (h, t) in ((0, 0), (3, 1023), (5, 1024), (11, 5000), (7, 20000), (2, 32767)):
        ro, rd = _row_ref(q, k, v, 0, h, t, M)
        e = (oc[0, t, h].double() - ro).abs().max().item() / ro.abs().max().item()
        assert e < TOL, ("o row", h, t, e)
        assert abs(denc[0, t, h].item() - rd) / rd < TOL, ("den row", h, t)
    # state rows p = g E^2 + a E + b for a few p, all value columns, two heads
    Sc = S.cpu()
    kd, vd = k.double(), v.double()
    for h in (0, 9):
        for p in (0, 17, 255, 256 + 3 * 16 + 5, 1023):
            gg, a_, b_ = p // 256, (p // 16) % 16, p % 16
            w = kd[0, :, h, 16 * gg + a_] * kd[0, :, h, 16 * gg + b_] * 0.25
            ref = (w[:, None] * vd[0, :, h]).sum(0)
            e = (Sc[0, h, p].double() - ref).abs().max().item() / ref.abs().max().item()
            assert e < TOL, ("S row", h, p, e)
    # decode at batch 64 from the broadcast prefill state
    Bd = 64
    Sd = S.expand(Bd, H, -1, -1).contiguous()
    zd = z.expand(Bd, H, -1).contiguous()
    S_ref = {bh: (S[0, bh[1]].cpu().double().clone(), z[0, bh[1]].cpu().double().clone())
             for bh in ((0, 0), (63, 11))}
    for i in range(3):
        gi = torch.Generator().manual_seed(4000 + i)
        qd, kd_, vd_ = ((torch.randn(Bd, H, 64, generator=gi) / 8).to(BF) for _ in range(3))
        od = S_.kata_decode_step(Sd, zd, qd.to(dev), kd_.to(dev), vd_.to(dev), num_groups=M)
        for (bb, hh) in S_ref:
            Sr, zr = S_ref[(bb, hh)]
            sl = lambda x: x[bb:bb + 1, hh:hh + 1]  # noqa: E731
            o_r, Sr, zr = K.kata_decode_step(Sr[None, None], zr[None, None], sl(qd), sl(kd_),
                                             sl(vd_), M)
            S_ref[(bb, hh)] = (Sr[0, 0], zr[0, 0])
            assert mar(od[bb, hh], o_r[0, 0]) < TOL, (i, bb, hh)


# ---------------------------------------------------------------------------
# packed state layout: one row per unordered pair a <= b of each group
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("M", [4, 2])
@pytest.mark.parametrize("case", [(2, 300, 2, 128), (1, 1000, 3, 256)],
                         ids=lambda c: "B{}T{}H{}L{}".format(*c))
def test_packed_prefill_equals_full(S_, M, case):
    """The packed-layout prefill runs the same kernels: o and den are
    bit-identical to the full-layout call's, and its state holds the full
    state's pair rows bit for bit (the scan writes one value to both rows of
    a pair).  Also continued in place from a packed state."""
    B, T, H, L = case
    print(f"packed prefill {case} M={M}", flush=True)
    dev = torch.device("cuda")
    q, k, v = (gen((B, T, H, 64), 60 + i + T).to(dev) for i in range(3))
    o, den, S, z = S_.kata_prefill(q, k, v, num_groups=M, seg_len=L)
    op, denp, Sp, zp = S_.kata_prefill(q, k, v, num_groups=M, seg_len=L, packed_state=True)
    PT = S_.state_rows(64, M, True)
    assert Sp.shape == (B, H, PT, 64) and zp.shape == (B, H, PT)
    assert torch.equal(o, op) and torch.equal(den, denp)
    Su, zu = S_.unpack_state(Sp, zp, M)
    assert torch.equal(Su, S) and torch.equal(zu, z)
    n = T // 3
    _, _, F1, y1 = S_.kata_prefill(q[:, :n], k[:, :n], v[:, :n], num_groups=M, seg_len=L)
    of, denf, F2, y2 = S_.kata_prefill(q[:, n:], k[:, n:], v[:, n:], num_groups=M, seg_len=L,
                                       initial_state=(F1, y1), in_place=True)
    _, _, P1, x1 = S_.kata_prefill(q[:, :n], k[:, :n], v[:, :n], num_groups=M, seg_len=L,
                                   packed_state=True)
    o2, den2, P2, x2 = S_.kata_prefill(q[:, n:], k[:, n:], v[:, n:], num_groups=M, seg_len=L,
                                       initial_state=(P1, x1), in_place=True, packed_state=True)
    assert P2.data_ptr() == P1.data_ptr() and x2.data_ptr() == x1.data_ptr()
    assert torch.equal(o2, of) and torch.equal(den2, denf)
    Su2, zu2 = S_.unpack_state(P2, x2, M)
    assert torch.equal(Su2, F2) and torch.equal(zu2, y2)


@pytest.mark.parametrize("M", [4, 2])
def test_packed_decode_equals_full(S_, M):
    """Decode steps on the packed state.  Its rows stay the full state's pair
    rows a <= b bit for bit.  The full layout forms a pair's two rows in two
    rounding orders, so those agree to float32 rounding.  o agrees with the
    full-layout step to one bf16 rounding (the readout sums each pair once,
    weighted 2 off the diagonal) and with the float64 oracle."""
    B, n, H, steps = 3, 200, 2, 4
    print(f"packed decode M={M}", flush=True)
    dev = torch.device("cuda")
    q, k, v = (gen((B, n + steps, H, 64), 91 + i) for i in range(3))
    _, _, S, z = S_.kata_prefill(q[:, :n].to(dev), k[:, :n].to(dev), v[:, :n].to(dev),
                                 num_groups=M, seg_len=128)
    Sp, zp = S_.pack_state(S, z, M)
    Sr, zr = S.cpu().double(), z.cpu().double()
    for i in range(steps):
        t = n + i
        x = [y[:, t].to(dev) for y in (q, k, v)]
        o = S_.kata_decode_step(S, z, *x, num_groups=M)
        op = S_.kata_decode_step(Sp, zp, *x, num_groups=M)
        o_ref, Sr, zr = K.kata_decode_step(Sr, zr, q[:, t], k[:, t], v[:, t], M)
        assert mar(op, o_ref) < TOL, (i, mar(op, o_ref))
        assert mar(op, o) < 8e-3, (i, mar(op, o))
        Sf, zf = S_.pack_state(S, z, M)
        assert torch.equal(Sf, Sp) and torch.equal(zf, zp), i
        Su, zu = S_.unpack_state(Sp, zp, M)
        assert mar(Su, S) < 1e-6 and mar(zu, z) < 1e-6, i


# ---------------------------------------------------------------------------
# decode cache (linatt_amd.kata_cache): prefill, continued prefill, decode
# steps, all against the flash forward over every token so far
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("M", [4, 2])
def test_cache_prefill_then_decode_equals_parallel(M):
    from linatt_amd import parallel_kata_attn as P
    from linatt_amd.kata_cache import parallel_kata_attn_cached
    B, H, n, steps = 2, 3, 300, 5
    T = n + steps
    q, k, v = gen((B, T, H, 64), 70), gen((B, T, H, 64), 71), gen((B, T, H, 64), 72)
    dev = torch.device("cuda")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o_par, _ = P.parallel_kata_attn_fwd(qd, kd, vd, num_groups=M)
    o_ref, _ = K.kata_fwd(q, k, v, M)
    o_pre, st = parallel_kata_attn_cached(qd[:, :n], kd[:, :n], vd[:, :n], None, M)
    assert st.offset == n
    assert mar(o_pre, o_ref[:, :n]) < TOL
    for i in range(steps):
        t = n + i
        o_t, st = parallel_kata_attn_cached(qd[:, t:t + 1], kd[:, t:t + 1], vd[:, t:t + 1], st, M)
        assert o_t.shape == (B, 1, H, 64) and st.offset == t + 1
        assert mar(o_t[:, 0], o_ref[:, t]) < TOL, i
        assert mar(o_t[:, 0], o_par[:, t].float()) < TOL, i
    # the state after all tokens equals the psi sums of every key (the cache
    # keeps the packed layout)
    from linatt_amd import spd_state as S_
    assert st.S.shape[2] == S_.state_rows(64, M, True)
    S_full, z_full = S_.unpack_state(st.S, st.z, M)
    S_ref, z_ref = K.kata_state_prefill(k, v, M)
    assert mar(S_full, S_ref) < TOL and mar(z_full, z_ref) < TOL


@pytest.mark.parametrize("split", [(200, 333), (128, 1), (1, 256), (1100, 500)])
def test_cache_continued_prefill(split):
    """Prefill of n1 tokens continued by a prefill of n2 (the scan starts from
    the cached state) equals one prefill of n1 + n2, outputs and state."""
    from linatt_amd.kata_cache import parallel_kata_attn_cached
    n1, n2 = split
    B, H, M = 1, 2, 4
    T = n1 + n2
    q, k, v = gen((B, T, H, 64), 73 + T), gen((B, T, H, 64), 74 + T), gen((B, T, H, 64), 75 + T)
    dev = torch.device("cuda")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o_all, st_all = parallel_kata_attn_cached(qd, kd, vd, None, M)
    o1, st = parallel_kata_attn_cached(qd[:, :n1], kd[:, :n1], vd[:, :n1], None, M)
    o2, st = parallel_kata_attn_cached(qd[:, n1:], kd[:, n1:], vd[:, n1:], st, M)
    assert st.offset == T
    o_ref, _ = K.kata_fwd(q, k, v, M)
    assert mar(torch.cat([o1, o2], 1), o_ref) < TOL
    assert mar(o2, o_all[:, n1:].float()) < TOL
    # the prefill forms segment states by MFMA from bf16-rounded psi features,
    # a one-token continuation (the decode step) adds fp32 products: the two
    # states agree to bf16 rounding, not bit for bit
    assert mar(st.S, st_all.S) < 2e-3 and mar(st.z, st_all.z) < 2e-3


def test_layer_cache_decode_loop():
    """Two mixer layers keeping their state through the fla-style helpers:
    a prompt, then three generated tokens, as an incremental generate() does."""
    from linatt_amd.kata_cache import (LayerStateCache, get_layer_cache, parallel_kata_attn_cached,
                                       update_layer_cache)

    class Layer:
        def __init__(self, i):
            self.layer_idx = i

    layers = [Layer(0), Layer(1)]
    B, H, n, M = 2, 2, 129, 4
    T = n + 3
    dev = torch.device("cuda")
    xs = [[gen((B, T, H, 64), 80 + 10 * li + j).to(dev) for j in range(3)] for li in range(2)]
    cache = LayerStateCache()
    outs = [[], []]
    for lo, hi in [(0, n), (n, n + 1), (n + 1, n + 2), (n + 2, n + 3)]:
        for layer, (q, k, v) in zip(layers, xs):
            last = get_layer_cache(layer, cache)
            rec = last["recurrent_state"] if last is not None else None
            o, fin = parallel_kata_attn_cached(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], rec, M)
            update_layer_cache(layer, cache, recurrent_state=fin, offset=hi - lo)
            outs[layer.layer_idx].append(o)
    assert cache.get_seq_length() == T
    for li, (q, k, v) in enumerate(xs):
        o_ref, _ = K.kata_fwd(q.cpu(), k.cpu(), v.cpu(), M)
        assert mar(torch.cat(outs[li], 1), o_ref) < TOL


def test_cache_paths_share_the_state():
    """A state from the state-form prefill (1100 tokens) continued by a chunk
    that the cache sends down the flash path (64 tokens over B H = 96 pairs),
    then decode steps on the state-form decode: every output equals the rows
    of the flash forward over all tokens."""
    from linatt_amd import parallel_kata_attn as P
    from linatt_amd.kata_cache import parallel_kata_attn_cached
    B, H, M = 32, 3, 4
    n0, n1, steps = 1100, 64, 2
    T = n0 + n1 + steps
    print(f"\ncache paths share the state: B{B} H{H} T{T}", flush=True)
    q, k, v = (gen((B, T, H, 64), 90 + i).cuda() for i in range(3))
    o_par, _ = P.parallel_kata_attn_fwd(q, k, v, num_groups=M)
    o0, st = parallel_kata_attn_cached(q[:, :n0], k[:, :n0], v[:, :n0], None, M)
    o1, st = parallel_kata_attn_cached(q[:, n0:n0 + n1], k[:, n0:n0 + n1], v[:, n0:n0 + n1], st, M)
    outs = [o0, o1]
    for t in range(n0 + n1, T):
        o, st = parallel_kata_attn_cached(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], st, M)
        outs.append(o)
    assert st.offset == T
    err = mar(torch.cat(outs, 1), o_par.float())
    print(f"  max rel err against the flash forward {err:.1e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("M,packed", [(4, True), (4, False), (2, True)])
def test_split_decode_step_equals_decode_step(M, packed):
    """``linatt_kata_decode_step_split`` (rows over several workgroups per
    (b, h), partials added by a second launch) against the one-workgroup
    decode step: S and z bit for bit, o to the rounding of the final sums."""
    from linatt_amd import _lib, spd_state as S_
    B, H, dk = 2, 5, 64
    L = _lib.load()
    R = S_.state_rows(dk, M, packed)
    nws = L.linatt_kata_decode_workspace_bytes(B, H, dk, M, int(packed))
    assert nws > 0
    print(f"\nsplit MFMA-path decode M{M} packed={packed} rows {R}", flush=True)
    S0 = (gen((B, H, R, 64), 600 + M, 0.05).float()).cuda()
    z0 = (gen((B, H, R), 601 + M).float().abs() + 0.5).cuda()
    q, k, v = (gen((B, H, 64), 602 + i, 0.5).cuda() for i in range(3))
    sc = 1.0 / (dk // M) ** 0.5
    outs = []
    for split in (False, True):
        S, z = S0.clone(), z0.clone()
        o = torch.empty(B, H, 64, device="cuda", dtype=BF)
        head = (_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(S), _lib.ptr(z), _lib.ptr(o))
        if split:
            ws = torch.empty(nws, device="cuda", dtype=torch.uint8)
            _lib.check("split", L.linatt_kata_decode_step_split(
                *head, _lib.ptr(ws), nws, B, H, dk, 64, M, int(packed), sc, 1e-6, 1, _lib.stream_of(q)))
        else:
            name = "linatt_kata_decode_step_packed" if packed else "linatt_kata_decode_step"
            _lib.check(name, getattr(L, name)(*head, B, H, dk, 64, M, sc, 1e-6, 1, _lib.stream_of(q)))
        outs.append((S, z, o))
    torch.cuda.synchronize()
    (S1, z1, o1), (S2, z2, o2) = outs
    assert torch.equal(S1, S2) and torch.equal(z1, z2)
    assert mar(o2, o1) < 1e-2
