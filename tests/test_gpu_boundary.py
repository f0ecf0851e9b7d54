"""GPU checks of the drop-in boundary and of run-to-run determinism at the
full BASELINE shapes.

* The reference's trainer runs the mixer under ``torch.autocast(bf16)`` with
  float32 master weights (``train_llm.py:424``): the projections hand bf16
  q/k/v (and, for the gated delta rule, bf16 gates) to the ops, and the
  gradients must reach the float32 leaves.  The ops are checked there against
  the float64 oracle on the exact tensors they received.
* Every kernel is deterministic (no atomics, fixed reduction order), so two
  runs on the same inputs must agree bit for bit on every head; a cross-wave
  LDS race shows up as a few heads that differ, which a per-head oracle
  check can miss.  Covered for KATA config 2 (fwd+bwd) and config 5 (prefill
  plus three decode steps); the delta rule has its own in
  ``test_gpu_delta.py``.
"""

import pytest
import torch

from oracle import delta as D
from oracle import kata as K

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def mar(x, ref):
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = ref.abs().max().item()
    return (x - ref).abs().max().item() / (den if den > 0 else 1.0)


def _proj_inputs(B, T, C, n_out, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, T, C, generator=g)).to(DEV).requires_grad_(True)
    W = (torch.randn(C, n_out, generator=g) / C ** 0.5).to(DEV).requires_grad_(True)
    return x, W


def test_kata_under_autocast_fp32_leaves():
    from linatt_amd import parallel_kata_attn as P
    B, T, H, D_, M, C = 2, 200, 3, 64, 4, 96
    x, W = _proj_inputs(B, T, C, 3 * H * D_, 70)
    do = torch.randn(B, T, H, D_, generator=torch.Generator().manual_seed(71)).to(DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        qkv = (x @ W) * 0.125
        q, k, v = (t.reshape(B, T, H, D_) for t in qkv.split(H * D_, dim=-1))
        assert q.dtype == torch.bfloat16
        for t in (q, k, v):
            t.retain_grad()
        o = P.parallel_kata_attn(q, k, v, num_groups=M)
    assert o.dtype == torch.bfloat16
    (o.float() * do).sum().backward()
    assert x.grad.dtype == torch.float32 and W.grad.dtype == torch.float32
    assert torch.isfinite(x.grad).all() and torch.isfinite(W.grad).all()
    qc, kc, vc = (t.detach().cpu() for t in (q, k, v))
    o_ref, den_ref = K.kata_fwd(qc, kc, vc, M)
    refs = K.kata_bwd(qc, kc, vc, o_ref, den_ref, do.cpu().to(torch.bfloat16), M)
    assert mar(o, o_ref) < 2e-2
    for name, t, ref in zip(("dq", "dk", "dv"), (q, k, v), refs):
        assert t.grad.dtype == torch.bfloat16
        assert mar(t.grad, ref) < 2e-2, name


def test_gated_delta_under_autocast_fp32_leaves():
    from linatt_amd import delta_rule as R
    B, T, H, K_, C = 2, 150, 2, 64, 64
    x, W = _proj_inputs(B, T, C, 3 * H * K_ + 2 * H, 72)
    do = torch.randn(B, T, H, K_, generator=torch.Generator().manual_seed(73)).to(DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = x @ W
        q, k, v, a, b = y.split([H * K_, H * K_, H * K_, H, H], dim=-1)
        q, k, v = (t.reshape(B, T, H, K_) for t in (q, k, v))
        g = torch.nn.functional.logsigmoid(a + 4) / 16
        beta = torch.sigmoid(b)
        for t in (q, k, v, g, beta):
            t.retain_grad()
        o, ht = R.chunk_gated_delta_rule(q, k, v, g, beta, output_final_state=True,
                                         use_qk_l2norm_in_kernel=True)
    assert o.dtype == torch.bfloat16 and ht.dtype == torch.float32
    (o.float() * do).sum().backward()
    assert x.grad.dtype == torch.float32 and torch.isfinite(x.grad).all()
    assert torch.isfinite(W.grad).all()
    ref = D.delta_rule_fwd_bwd(*(t.detach().cpu() for t in (q, k, v, beta, g)),
                               do=do.cpu().to(torch.bfloat16), use_qk_l2norm=True)
    assert mar(o, ref["o"]) < 2e-2
    assert mar(ht, ref["ht"]) < 2e-2
    for name, t in (("dq", q), ("dk", k), ("dv", v), ("dbeta", beta), ("dg", g)):
        assert t.grad.dtype == t.dtype, name
        assert mar(t.grad, ref[name]) < 2e-2, name


def test_kata_config2_repeat_runs_identical():
    from linatt_amd import parallel_kata_attn as P
    B, T, H, D_, M = 8, 2048, 12, 64, 4
    g = torch.Generator().manual_seed(1)
    q, k, v = ((torch.randn(B, T, H, D_, generator=g) / 8).to(torch.bfloat16).to(DEV)
               for _ in range(3))
    do = torch.randn(B, T, H, D_, generator=g).to(torch.bfloat16).to(DEV)
    scale = K.default_scale(D_, M)
    first = None
    for _ in range(2):
        o, den = P.parallel_kata_attn_fwd(q, k, v, M)
        grads = P.parallel_kata_attn_bwd(q, k, v, o, den, do, M, scale)
        out = [t.clone() for t in (o, den) + tuple(grads)]
        if first is None:
            first = out
            continue
        for name, a, b in zip(("o", "den", "dq", "dk", "dv"), first, out):
            assert torch.equal(a, b), name


def test_kata_config5_repeat_runs_identical():
    from linatt_amd import spd_state as S_
    H, D_, M, T, nb = 12, 64, 4, 32768, 64
    g = torch.Generator().manual_seed(4)
    q, k, v = ((torch.randn(1, T, H, D_, generator=g) / 8).to(torch.bfloat16).to(DEV)
               for _ in range(3))
    steps = []
    for i in range(3):
        gi = torch.Generator().manual_seed(4000 + i)
        steps.append([(torch.randn(nb, H, D_, generator=gi) / 8).to(torch.bfloat16).to(DEV)
                      for _ in range(3)])
    first = None
    for _ in range(2):
        o, den, S, z = S_.kata_prefill(q, k, v, num_groups=M)
        S = S.expand(nb, -1, -1, -1).contiguous()
        z = z.expand(nb, -1, -1).contiguous()
        outs = [o.clone(), den.clone()]
        for qs, ks, vs in steps:
            outs.append(S_.kata_decode_step(S, z, qs, ks, vs, num_groups=M).clone())
        outs += [S, z]
        if first is None:
            first = outs
            continue
        for i, (a, b) in enumerate(zip(first, outs)):
            assert torch.equal(a, b), i
