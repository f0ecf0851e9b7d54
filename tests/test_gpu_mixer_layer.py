"""The mixer harness: a minimal ``KataAttention.forward`` (``kata/layer.py:286-545``)
built from this build's ops, against the same layer in float64 from the oracle.

The harness keeps the reference layer's order of operations:
- q/k/v projections, the three short convolutions with SiLU (``:296-318``);
- per-head RMSNorm on q and k, then RoPE (``:340-372``);
- the flash branch, which calls ``parallel_kata_attn`` when a gradient is
  needed and ``parallel_kata_attn_fwd`` otherwise (the ``grad_on`` choice,
  ``:438-440, 456-487``), or the delta branch: beta from ``b_proj``, and q, k,
  v, beta padded to a power of two of at least 64 before ``flash_delta``
  (``:377-420``);
- the output RMSNorm and ``o_proj`` (``:539-541``).

The ``flash_M4_fused`` case runs the q and k chains (convolution, RMSNorm,
rotation) through ``fused_qk_prologue`` instead of the three modules, against
the same float64 layer.

It runs under ``torch.autocast(bf16)`` with float32 parameters and input, as
``train_llm.py:424`` runs the model.  The output and every gradient (input,
projections, convolution and norm weights) meet the bf16 bar of 2e-2
max-abs-relative against the float64 layer (measured: at most 1.4e-2),
although autocast rounds every projection output to bf16 and the float64
layer does not.
"""

import pytest
import torch
from torch import nn

from oracle import delta_kata as DK
from oracle import kata as K
from oracle import mixer as X

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
BAR = 2e-2


def mar(x, ref):
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = ref.abs().max().item()
    return (x - ref).abs().max().item() / (den if den > 0 else 1.0)


class MiniMixer(nn.Module):
    """The flash or delta branch of the reference mixer, through linatt_amd."""

    def __init__(self, hidden, H, D, M, branch, conv=4, fused=False):
        super().__init__()
        from linatt_amd.mixer import RMSNorm, RotaryEmbedding, ShortConvolution
        self.H, self.D, self.M, self.branch, self.fused = H, D, M, branch, fused
        self.q_proj = nn.Linear(hidden, H * D, bias=False)
        self.k_proj = nn.Linear(hidden, H * D, bias=False)
        self.v_proj = nn.Linear(hidden, H * D, bias=False)
        self.b_proj = nn.Linear(hidden, H, bias=False)
        self.o_proj = nn.Linear(H * D, hidden, bias=False)
        self.q_conv1d = ShortConvolution(H * D, conv, activation="silu")
        self.k_conv1d = ShortConvolution(H * D, conv, activation="silu")
        self.v_conv1d = ShortConvolution(H * D, conv, activation="silu")
        self.q_norm = RMSNorm(D, dtype=torch.float32)
        self.k_norm = RMSNorm(D, dtype=torch.float32)
        self.rotary = RotaryEmbedding(D)
        self.norm = RMSNorm(D, dtype=torch.float32)
        with torch.no_grad():  # non-trivial norm weights
            for m in (self.q_norm, self.k_norm, self.norm):
                m.weight.uniform_(0.75, 1.25)

    def forward(self, x):
        from linatt_amd.flash_delta import flash_delta
        from linatt_amd.parallel_kata_attn import parallel_kata_attn, parallel_kata_attn_fwd
        from linatt_amd.mixer import fused_qk_prologue
        B, T, _ = x.shape
        v, _ = self.v_conv1d(self.v_proj(x))
        v = v.reshape(B, T, self.H, self.D)
        if self.fused:
            q, _ = fused_qk_prologue(self.q_proj(x), self.q_conv1d, self.q_norm, self.rotary, self.D)
            k, _ = fused_qk_prologue(self.k_proj(x), self.k_conv1d, self.k_norm, self.rotary, self.D)
        else:
            q, _ = self.q_conv1d(self.q_proj(x))
            k, _ = self.k_conv1d(self.k_proj(x))
            q, k = (t.reshape(B, T, self.H, self.D) for t in (q, k))
            q, k = self.q_norm(q), self.k_norm(k)
            q, k = self.rotary(q, k)
        if self.branch == "flash":
            grad_on = torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v))
            if grad_on:
                o = parallel_kata_attn(q, k, v, num_groups=self.M)
            else:
                o, _ = parallel_kata_attn_fwd(q, k, v, num_groups=self.M)
        else:
            beta = torch.sigmoid(self.b_proj(x))
            Tp = max(64, 1 << (T - 1).bit_length())
            qh, kh, vh, bh = (t.contiguous() for t in (q, k, v, beta))
            if Tp != T:
                p = Tp - T
                qh, kh, vh = (nn.functional.pad(t, (0, 0, 0, 0, 0, p)) for t in (qh, kh, vh))
                bh = nn.functional.pad(bh, (0, 0, 0, p))
            o = flash_delta(qh.bfloat16(), kh.bfloat16(), vh.bfloat16(), bh.bfloat16(), self.M)
            o = o[:, :T].to(v.dtype)
        o = self.norm(o).reshape(B, T, self.H * self.D)
        return self.o_proj(o)

    def reference(self, x):
        """The same layer in float64 on the CPU from the oracle's functions."""
        P = {n: p.detach().double().cpu().requires_grad_(True) for n, p in self.named_parameters()}
        x = x.detach().double().cpu().requires_grad_(True)
        B, T, _ = x.shape

        def branch(name):
            y = x @ P[f"{name}_proj.weight"].T
            y, _ = X.short_conv(y, P[f"{name}_conv1d.weight"], None, "silu")
            return y.reshape(B, T, self.H, self.D)

        q, k, v = branch("q"), branch("k"), branch("v")
        q = X.rmsnorm(q, P["q_norm.weight"], 1e-5)
        k = X.rmsnorm(k, P["k_norm.weight"], 1e-5)
        q, k = X.rope(q, self.D), X.rope(k, self.D)
        if self.branch == "flash":
            o, _ = K.kata_fwd(q, k, v, self.M)
        else:
            beta = torch.sigmoid(x @ P["b_proj.weight"].T)
            o = DK.flash_delta_fwd(q, k, v, beta, self.M)[0]
        o = X.rmsnorm(o, P["norm.weight"], 1e-5).reshape(B, T, self.H * self.D)
        return o @ P["o_proj.weight"].T, x, P


@pytest.mark.parametrize("branch,T,M,fused", [("flash", 200, 4, False), ("delta", 100, 1, False),
                                              ("flash", 200, 4, True)],
                         ids=["flash_M4", "delta_M1_padded", "flash_M4_fused"])
def test_mixer_layer_under_autocast(branch, T, M, fused):
    torch.manual_seed(0)
    B, hidden, H, D = 2, 256, 4, 64
    layer = MiniMixer(hidden, H, D, M, branch, fused=fused).to(DEV)
    x = torch.randn(B, T, hidden, generator=torch.Generator().manual_seed(1)).to(DEV)
    dy = torch.randn(B, T, hidden, generator=torch.Generator().manual_seed(2)).to(DEV)
    xg = x.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = layer(xg)
    assert y.dtype == torch.bfloat16 and y.shape == (B, T, hidden)
    y.float().backward(dy)

    y_ref, x_ref, P_ref = layer.reference(x)
    (y_ref * dy.double().cpu()).sum().backward()
    print(f"\nmixer {branch}: y {mar(y, y_ref):.2e} dx {mar(xg.grad, x_ref.grad):.2e}", flush=True)
    assert mar(y, y_ref) < BAR
    assert mar(xg.grad, x_ref.grad) < BAR
    for name, p in layer.named_parameters():
        if branch == "flash" and name == "b_proj.weight":
            assert p.grad is None  # the flash branch does not use beta
            continue
        assert p.grad is not None and p.grad.dtype == torch.float32, name
        e = mar(p.grad, P_ref[name].grad)
        print(f"  d{name} {e:.2e}", flush=True)
        assert e < BAR, (name, e)

    if branch == "flash":
        # grad_on = False takes the no-grad forward: the same kernel, so the
        # same output bit for bit
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            y_ng = layer(x)
        assert torch.equal(y_ng, y.detach())


# ---------------------------------------------------------------------------
# The fused KataAttention.forward installed by linatt_amd.patch.apply_mixer(),
# on a module with the reference mixer's attribute layout
# ---------------------------------------------------------------------------


@pytest.fixture
def hooked(monkeypatch):
    import sys
    import types
    import mixer_layout
    from linatt_amd import patch

    class KataAttention(mixer_layout.KataAttentionLayout):
        pass

    layer_mod = types.ModuleType("kata.layer")
    layer_mod.KataAttention = KataAttention
    monkeypatch.setitem(sys.modules, "kata", types.ModuleType("kata"))
    monkeypatch.setitem(sys.modules, "kata.layer", layer_mod)
    assert patch.apply_mixer()
    yield KataAttention
    patch.restore()


HOOK_CASES = {
    "concat_M4": dict(M=4),
    "concat_M2_gqa": dict(M=2, num_kv_heads=2),
    "sum_M2_l2_ropegroup": dict(M=2, feature_map="kata_quadratic_sum", norm_q="l2", norm_k="l2",
                                rope_group=True),
    "concat_M2_decay": dict(M=2, use_decay=True),
    "concat_M2_offset_gate": dict(M=2, use_offset_gate=True),
}


@pytest.mark.parametrize("case", list(HOOK_CASES))
def test_hooked_mixer_under_autocast(hooked, case):
    """Output and every gradient through the fused forward within 2e-2 of
    the float64 layer."""
    import mixer_layout
    kw = dict(HOOK_CASES[case])
    M = kw.pop("M")
    torch.manual_seed(0)
    B, T, hidden, H, D = 2, 200, 256, 4, 64
    layer = hooked(hidden, H, D, M, **kw).to(DEV)
    x = torch.randn(B, T, hidden, generator=torch.Generator().manual_seed(1)).to(DEV)
    dy = torch.randn(B, T, hidden, generator=torch.Generator().manual_seed(2)).to(DEV)
    xg = x.clone().requires_grad_(True)
    print(f"\nhooked mixer {case}", flush=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y, _, _ = layer(xg)
    assert layer.original_calls == 0
    assert y.dtype == torch.bfloat16 and y.shape == (B, T, hidden)
    y.float().backward(dy)
    y_ref, x_ref, P_ref = mixer_layout.layout_reference(layer, x)
    (y_ref * dy.double().cpu()).sum().backward()
    print(f"  y {mar(y, y_ref):.2e} dx {mar(xg.grad, x_ref.grad):.2e}", flush=True)
    assert mar(y, y_ref) < BAR
    assert mar(xg.grad, x_ref.grad) < BAR
    for name, p in layer.named_parameters():
        assert p.grad is not None, name
        e = mar(p.grad, P_ref[name].grad)
        print(f"  d{name} {e:.2e}", flush=True)
        assert e < BAR, (name, e)


@pytest.mark.parametrize("M", [4, 2])
def test_hooked_mixer_prefill_then_decode_equals_parallel(hooked, M):
    """Prefill 150 tokens and decode 10 more one at a time through the hook
    with a LayerStateCache: the outputs equal the same layer's parallel
    forward over all 160 tokens (convolution, rotation and attention states
    carried across calls)."""
    from linatt_amd.kata_cache import LayerStateCache
    torch.manual_seed(3)
    B, T, P0, hidden, H, D = 2, 160, 150, 256, 4, 64
    layer = hooked(hidden, H, D, M).to(DEV)
    x = torch.randn(B, T, hidden, generator=torch.Generator().manual_seed(4)).to(DEV)
    print(f"\nhooked decode M{M}", flush=True)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        y_par, _, _ = layer(x)
        cache = LayerStateCache()
        outs = [layer(x[:, :P0], past_key_values=cache, use_cache=True)[0]]
        for t in range(P0, T):
            outs.append(layer(x[:, t:t + 1], past_key_values=cache, use_cache=True)[0])
    y_inc = torch.cat(outs, dim=1)
    assert layer.original_calls == 0 and cache.get_seq_length(0) == T
    e_pre, e_dec = mar(y_inc[:, :P0], y_par[:, :P0]), mar(y_inc[:, P0:], y_par[:, P0:])
    print(f"  prefill {e_pre:.2e} decode {e_dec:.2e}", flush=True)
    assert e_pre < BAR and e_dec < BAR


@pytest.mark.parametrize("kw", [dict(M=2, feature_map="kata_quadratic_sum"), dict(M=2, use_decay=True),
                                dict(M=1), dict(M=2, use_offset_gate=True)],
                         ids=["sum_M2", "decay_M2", "concat_M1", "offset_gate_M2"])
def test_hooked_mixer_decode_every_flash_score(hooked, kw):
    """The sum, decayed, one-group and offset-gated mixers decode from a
    state too: prefill + decode through the hook equals the parallel
    forward."""
    from linatt_amd.kata_cache import LayerStateCache
    kw = dict(kw)
    M = kw.pop("M")
    torch.manual_seed(5)
    B, T, P0, hidden, H, D = 2, 140, 130, 256, 4, 64
    layer = hooked(hidden, H, D, M, **kw).to(DEV)
    x = torch.randn(B, T, hidden, generator=torch.Generator().manual_seed(6)).to(DEV)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        y_par, _, _ = layer(x)
        cache = LayerStateCache()
        outs = [layer(x[:, :P0], past_key_values=cache, use_cache=True)[0]]
        for t in range(P0, T):
            outs.append(layer(x[:, t:t + 1], past_key_values=cache, use_cache=True)[0])
    y_inc = torch.cat(outs, dim=1)
    assert layer.original_calls == 0
    e = mar(y_inc, y_par)
    print(f"\nhooked decode {kw}: {e:.2e}", flush=True)
    assert e < BAR
