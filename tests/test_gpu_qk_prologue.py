"""The fused q/k prologue (``linatt_qk_prologue_fwd`` / ``_bwd``) against the
float64 chain of the oracle's pinned pieces: ``oracle.mixer.short_conv``,
``rmsnorm`` or ``oracle.delta.l2norm`` over each head, ``oracle.mixer.rope``
over rows of ``rope_width`` dims -- the order ``kata/layer.py:305-372`` runs
the three modules in.  Output, final convolution cache and every gradient
(x, conv weight and bias, norm weight) meet the dtype's bar (2e-2 for 16-bit,
1e-4 for fp32, max-abs-relative).  The cases cover the mixer's two rotations
(interleaved over the head, ``kata/layer.py:142-148``; half-split over each
E-dim group under ``rope_group``, ``:135-139, 356-368``), both norms
(``norm_q: rmsnorm | l2``), a partial rotation with pass-through dims,
ragged T, a decode cache and position offsets.  In fp32 the op also agrees
with the three linatt_amd modules run one after another (1e-5), and decoding
token by token from the cache reproduces the full forward's rows."""

import pytest
import torch

from oracle import delta as DL
from oracle import mixer as X

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
BAR = {torch.bfloat16: 2e-2, torch.float16: 2e-2, torch.float32: 1e-4}


def mar(x, ref):
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = ref.abs().max().item()
    return (x - ref).abs().max().item() / (den if den > 0 else 1.0)


def ref_chain(x, w, b, nw, cache, H, D, act, norm, eps, rw, rot, base, offset, inter):
    y, fc = X.short_conv(x, w, b, act, cache)
    B, T, _ = y.shape
    y = y.reshape(B, T, H, D)
    if norm == "rmsnorm":
        y = X.rmsnorm(y, nw, eps)
    elif norm == "l2":
        y = DL.l2norm(y, eps)
    if rot:
        y = X.rope(y.reshape(B, T, H * D // rw, rw), rot, base, offset, inter).reshape(B, T, H, D)
    return y, fc


# (dtype, B, T, H, D, W, bias, norm, norm weight, rope_width, rot_dim, interleaved, offset, cache)
CASES = [
    (torch.bfloat16, 2, 200, 4, 64, 4, False, "rmsnorm", True, 64, 64, True, 0, False),
    (torch.bfloat16, 2, 77, 4, 64, 4, True, "l2", False, 16, 16, False, 0, False),
    (torch.float32, 1, 50, 3, 128, 3, False, "rmsnorm", False, 128, 0, True, 0, True),
    (torch.float16, 2, 33, 2, 32, 2, True, "rmsnorm", True, 32, 16, False, 5, True),
    (torch.bfloat16, 3, 1, 2, 64, 4, False, None, False, 64, 64, True, 100, True),
    (torch.float32, 2, 129, 6, 64, 4, True, "rmsnorm", True, 64, 62, True, 7, False),
]
IDS = ["bf16_rms_interleaved", "bf16_l2_rope_group", "fp32_D128_norope_cache",
       "fp16_partial_halfsplit_offset", "bf16_decode_T1", "fp32_rot62_H6"]


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_qk_prologue_matches_oracle(case):
    from linatt_amd.mixer import qk_prologue
    dt, B, T, H, D, W, has_b, norm, has_nw, rw, rot, inter, off, has_cache = case
    C = H * D
    g = torch.Generator().manual_seed(CASES.index(case))
    x = torch.randn(B, T, C, generator=g)
    w = torch.randn(C, 1, W, generator=g) / W ** 0.5
    b = torch.randn(C, generator=g) * 0.2 if has_b else None
    nw = torch.empty(D).uniform_(0.75, 1.25, generator=g) if has_nw else None
    cache = torch.randn(B, C, W, generator=g).to(dt) if has_cache else None
    dy = torch.randn(B, T, H, D, generator=g)
    eps = 1e-6 if norm == "l2" else 1e-5
    base = 10000.0

    xd = x.to(dt).to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    bd = b.to(DEV).requires_grad_(True) if b is not None else None
    nwd = nw.to(DEV).requires_grad_(True) if nw is not None else None
    print(f"\ncase {case}", flush=True)
    y, fc = qk_prologue(xd, wd, bd, head_dim=D, norm=norm, norm_weight=nwd, eps=eps,
                        rot_dim=rot, rope_width=rw, base=base, offset=off, interleaved=inter,
                        cache=cache.to(DEV) if cache is not None else None,
                        output_final_state=True)
    assert y.shape == (B, T, H, D) and y.dtype == dt
    y.backward(dy.to(dt).to(DEV))

    xr = x.to(dt)  # the rounded input both sides see
    y_ref, grads = X.fwd_bwd(
        lambda xx, ww, bb, nn_: ref_chain(xx, ww, bb, nn_, cache, H, D, "silu", norm, eps,
                                          rw, rot, base, off, inter)[0],
        [xr, w, b, nw], dy)
    _, fc_ref = ref_chain(xr, w, b, nw, cache, H, D, "silu", norm, eps, rw, rot, base, off, inter)
    bar = BAR[dt]
    errs = {"y": mar(y, y_ref), "dx": mar(xd.grad, grads[0]), "dw": mar(wd.grad, grads[1])}
    if b is not None:
        errs["db"] = mar(bd.grad, grads[2])
    if nw is not None:
        errs["dnw"] = mar(nwd.grad, grads[3])
    print("  " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v < bar, (k, v)
    # the cache holds inputs, copied without arithmetic
    assert torch.equal(fc.cpu(), fc_ref.to(dt))


def _chain_modules(dt, H, D, inter, rw, norm):
    from linatt_amd.mixer import RMSNorm, RotaryEmbedding, ShortConvolution
    torch.manual_seed(3)
    conv = ShortConvolution(H * D, 4, bias=True).to(DEV)
    nrm = RMSNorm(D, dtype=torch.float32).to(DEV) if norm == "rmsnorm" else norm
    if isinstance(nrm, RMSNorm):
        with torch.no_grad():
            nrm.weight.uniform_(0.75, 1.25)
    rot = RotaryEmbedding(rw, interleaved=inter)
    return conv, nrm, rot


@pytest.mark.parametrize("norm,inter,rw", [("rmsnorm", True, 64), ("l2", False, 16)],
                         ids=["rms_full_interleaved", "l2_group16"])
def test_qk_prologue_matches_unfused_modules_fp32(norm, inter, rw):
    """fp32: the fused op against ShortConvolution -> RMSNorm / l2norm ->
    RotaryEmbedding from linatt_amd, outputs and every gradient."""
    from linatt_amd.delta_rule import l2norm as l2
    from linatt_amd.mixer import fused_qk_prologue
    B, T, H, D = 2, 97, 3, 64
    conv, nrm, rot = _chain_modules(torch.float32, H, D, inter, rw, norm)
    x = torch.randn(B, T, H * D, device=DEV)
    dy = torch.randn(B, T, H, D, device=DEV)
    params = [p for p in list(conv.parameters()) + (list(nrm.parameters()) if norm == "rmsnorm" else [])]

    def unfused(xx):
        u, _ = conv(xx)
        u = u.view(B, T, H, D)
        u = nrm(u) if norm == "rmsnorm" else l2(u)
        ug = u.reshape(B, T, H * D // rw, rw)
        a, _ = rot(ug, ug)
        return a.reshape(B, T, H, D)

    out = []
    for fn in (lambda xx: fused_qk_prologue(xx, conv, nrm, rot, D)[0], unfused):
        for p in params:
            p.grad = None
        xx = x.clone().requires_grad_(True)
        y = fn(xx)
        y.backward(dy)
        out.append([y.detach(), xx.grad] + [p.grad.clone() for p in params])
    for a, r in zip(*out):
        assert mar(a, r) < 1e-5, mar(a, r)


def test_qk_prologue_decode_matches_full_forward():
    """Prefill of T0 tokens with the cache out, then single-token steps with
    the cache and position offsets: the rows equal the full forward's."""
    from linatt_amd.mixer import qk_prologue
    B, T, T0, H, D = 2, 40, 33, 2, 64
    torch.manual_seed(5)
    x = torch.randn(B, T, H * D, device=DEV)
    w = torch.randn(H * D, 1, 4, device=DEV) / 2
    nw = torch.rand(D, device=DEV) + 0.5
    kw = dict(head_dim=D, norm="rmsnorm", norm_weight=nw, interleaved=True)
    full, _ = qk_prologue(x, w, **kw)
    y0, cache = qk_prologue(x[:, :T0], w, output_final_state=True, **kw)
    rows = [y0]
    for t in range(T0, T):
        yt, cache = qk_prologue(x[:, t:t + 1], w, offset=t, cache=cache, output_final_state=True,
                                **kw)
        rows.append(yt)
    assert mar(torch.cat(rows, 1), full) < 1e-6


def test_qk_prologue_repeat_runs_identical():
    """Fixed-order reductions: two runs give the same bits, gradients included."""
    from linatt_amd.mixer import qk_prologue
    B, T, H, D = 4, 1000, 12, 64
    torch.manual_seed(6)
    x = torch.randn(B, T, H * D, device=DEV, dtype=torch.bfloat16)
    w = (torch.randn(H * D, 1, 4, device=DEV) / 2).requires_grad_(True)
    nw = (torch.rand(D, device=DEV) + 0.5).requires_grad_(True)
    dy = torch.randn(B, T, H, D, device=DEV, dtype=torch.bfloat16)
    res = []
    for _ in range(2):
        w.grad = nw.grad = None
        xx = x.clone().requires_grad_(True)
        y, _ = qk_prologue(xx, w, head_dim=D, norm="rmsnorm", norm_weight=nw)
        y.backward(dy)
        res.append([y, xx.grad, w.grad.clone(), nw.grad.clone()])
    for a, b in zip(*res):
        assert torch.equal(a, b)
