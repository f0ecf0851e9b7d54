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
``kataconv_cat_l2_gdn_340m`` mixer).
"""

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
