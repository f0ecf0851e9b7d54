"""The hot-path operators inside HIP graphs (``torch.cuda.CUDAGraph``).

Captured: a KATA training step (concat score, forward + backward through
``parallel_kata_attn``), the gated delta rule forward + backward with an
initial state, a loop of four decode steps on the psi-state, and the decode
cache of the flash scores outside the MFMA state form (a prefill from an
empty cache, four decode steps and a continued prefill, through
``kata_cache.parallel_kata_attn_cached`` and the ``linatt_kata_gen_*``
kernels).  Each
graph is replayed three times, with unrelated eager work and a host
synchronisation before every replay, and each replay must reproduce the
eager result bit for bit: the kernels are deterministic, so any difference
would come from the capture itself (a recorded memset, a host-side
allocation or copy, work on a stream outside the capture).

The backward is driven with ``torch.autograd.backward`` on the outputs and
their upstream gradients, so the graphs hold the library's kernels and
torch's own allocations, but no reduction of torch's.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def gen(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32) * std


def _eager_noise(i):
    """Unrelated eager work and a host synchronisation between replays."""
    x = torch.randn(257 + i, 129, device="cuda")
    y = torch.relu(x) * 3 + x.roll(1, 0)
    torch.cuda.synchronize()
    return y


def _capture(step):
    """Warm ``step`` up on a side stream, then capture it; returns the graph
    and the (graph-owned) tensors the captured call returned."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = step()
    torch.cuda.synchronize()
    return g, out


def _replay_and_check(g, out, ref, names, reset=None):
    for r in range(3):
        _eager_noise(r)
        if reset is not None:
            reset()
        g.replay()
        torch.cuda.synchronize()
        print(f"replay {r}", flush=True)
        for name, a, b in zip(names, out, ref):
            assert torch.equal(a, b), (r, name, (a.float() - b.float()).abs().max().item())


def test_kata_training_step_graph():
    from linatt_amd import parallel_kata_attn as P
    B, T, H, D, M = 2, 300, 4, 64, 4
    print(f"\nKATA concat B{B} T{T} H{H} M{M} in a graph", flush=True)
    q, k, v = (gen((B, T, H, D), 11 + i, 0.125).to(BF).cuda().requires_grad_(True) for i in range(3))
    do = gen((B, T, H, D), 14).to(BF).cuda()

    def step():
        for x in (q, k, v):
            x.grad = None
        o = P.parallel_kata_attn(q, k, v, num_groups=M)
        torch.autograd.backward([o], [do])
        return o, q.grad, k.grad, v.grad

    ref = [t.detach().clone() for t in step()]
    torch.cuda.synchronize()
    g, out = _capture(step)
    _replay_and_check(g, out, ref, ("o", "dq", "dk", "dv"))


def test_gated_delta_rule_graph():
    from linatt_amd import delta_rule as R
    B, T, H, K = 2, 200, 2, 64
    print(f"\ngated delta rule B{B} T{T} H{H} K=V={K} in a graph", flush=True)
    q = gen((B, T, H, K), 21).to(BF).cuda().requires_grad_(True)
    k = torch.nn.functional.normalize(gen((B, T, H, K), 22), dim=-1).to(BF).cuda().requires_grad_(True)
    v = gen((B, T, H, K), 23).to(BF).cuda().requires_grad_(True)
    beta = torch.sigmoid(gen((B, T, H), 24)).cuda().requires_grad_(True)
    gt = (torch.nn.functional.logsigmoid(gen((B, T, H), 25) + 4) / 16).cuda().requires_grad_(True)
    h0 = gen((B, H, K, K), 26, 0.02).cuda().requires_grad_(True)
    do = gen((B, T, H, K), 27).to(BF).cuda()
    dht = gen((B, H, K, K), 28).cuda()
    leaves = (q, k, v, beta, gt, h0)

    def step():
        for x in leaves:
            x.grad = None
        o, ht = R.chunk_gated_delta_rule(q, k, v, gt, beta, initial_state=h0, output_final_state=True)
        torch.autograd.backward([o, ht], [do, dht])
        return (o, ht) + tuple(x.grad for x in leaves)

    names = ("o", "ht", "dq", "dk", "dv", "dbeta", "dg", "dh0")
    ref = [t.detach().clone() for t in step()]
    torch.cuda.synchronize()
    g, out = _capture(step)
    _replay_and_check(g, out, ref, names)


def test_decode_loop_graph():
    from linatt_amd import spd_state as S_
    B, H, M, n = 4, 2, 4, 4
    P = M * 16 * 16
    print(f"\n{n} decode steps B{B} H{H} M{M} in a graph", flush=True)
    S0 = gen((B, H, P, 64), 31, 0.05).cuda()
    z0 = gen((B, H, P), 32).abs().cuda()
    steps = [tuple(gen((B, H, 64), 40 + 3 * i + j, 0.25).to(BF).cuda() for j in range(3))
             for i in range(n)]
    S, z = S0.clone(), z0.clone()

    def loop():
        return [S_.kata_decode_step(S, z, *x, num_groups=M) for x in steps]

    ref = [o.clone() for o in loop()] + [S.clone(), z.clone()]
    torch.cuda.synchronize()
    g, outs = _capture(loop)

    def reset():
        S.copy_(S0)
        z.copy_(z0)

    _replay_and_check(g, list(outs) + [S, z], ref,
                      tuple(f"o{i}" for i in range(n)) + ("S", "z"), reset)


@pytest.mark.parametrize("variant,M,decay", [("sum", 4, False), ("concat", 1, True)])
def test_generic_cache_graph(variant, M, decay):
    from linatt_amd.kata_cache import parallel_kata_attn_cached
    B, H, dk = 2, 3, 64
    splits = [0, 70, 71, 72, 73, 74, 104]
    T = splits[-1]
    print(f"\ngeneric cache in a graph: {variant} M{M} decay={decay} B{B} H{H} T{T}", flush=True)
    q = gen((B, T, H, dk), 60, 0.5).to(BF).cuda()
    k = gen((B, T, H, dk), 61, 0.5).to(BF).cuda()
    v = gen((B, T, H, 64), 62).to(BF).cuda()
    c = -(gen((B, T, H), 63).abs() * 0.05).cumsum(1).cuda() if decay else None

    def cc(s, e):
        if c is None:
            return None
        return (c[:, s:e] - (c[:, s - 1:s] if s > 0 else 0.0)).contiguous()

    def run():
        st, outs = None, []
        for s, e in zip(splits[:-1], splits[1:]):
            o, st = parallel_kata_attn_cached(q[:, s:e], k[:, s:e], v[:, s:e], st, M, None,
                                              variant=variant, c=cc(s, e))
            outs.append(o)
        return outs + [st.S, st.z]

    ref = [t.clone() for t in run()]
    torch.cuda.synchronize()
    g, out = _capture(run)
    _replay_and_check(g, out, ref, tuple(f"o{i}" for i in range(len(splits) - 1)) + ("S", "z"))
