"""Host-side boundary checks that need no GPU: the run-time rebinding hook
(``linatt_amd.patch``, after the reference's ``fla_patches.py:19-31, 195-200``)
and argument validation that must raise before any device work."""

import sys
import types

import pytest
import torch

from linatt_amd import delta_rule, parallel_kata_attn, patch, spd_state


def _stub(name, **attrs):
    m = types.ModuleType(name)
    for k, v in attrs.items():
        setattr(m, k, v)
    return m


def _orig(tag):
    def f(*a, **k):
        return tag
    f.__name__ = tag
    return f


MIXER_NAMES = ("ShortConvolution", "RMSNorm", "RotaryEmbedding")
DELTA_KATA_NAMES = ("flash_delta", "flash_delta_U", "flash_delta_readout", "flash_delta_den")
KATA_NAMES = ("parallel_kata_attn", "parallel_kata_attn_fwd", "parallel_kata_attn_sum",
              "parallel_kata_attn_sum_fwd_impl", "parallel_kata_attn_decay",
              "parallel_kata_attn_bwd", "parallel_kata_attn_bwd_triton")


@pytest.fixture
def stub_reference(monkeypatch):
    """The reference's modules as stubs in sys.modules: kata.layer imports the
    KATA ops by name (kata/layer.py:29-37), fla's layers import the delta ops
    by name."""
    mods = {
        "kata": _stub("kata"),
        "kata.parallel_kata_attn": _stub("kata.parallel_kata_attn", **{n: _orig("ref_" + n) for n in KATA_NAMES}),
        # the mixer binds a subset of the names (no backward entry points)
        "kata.layer": _stub("kata.layer", **{n: _orig("layer_" + n)
                                              for n in KATA_NAMES[:5] + MIXER_NAMES + ("flash_delta",)}),
        "kata.spd": _stub("kata.spd"),
        "kata.spd.chunk_scan_cat": _stub("kata.spd.chunk_scan_cat", spd_chunk_scan_cat=_orig("ref_scan")),
        "kata.spd.flash_delta": _stub("kata.spd.flash_delta",
                                      **{n: _orig("ref_" + n) for n in DELTA_KATA_NAMES}),
        "fla": _stub("fla"),
        "fla.layers": _stub("fla.layers"),
        "fla.layers.delta_net": _stub("fla.layers.delta_net", chunk_delta_rule=_orig("fla_dn")),
        "fla.layers.gated_deltanet": _stub("fla.layers.gated_deltanet",
                                           chunk_gated_delta_rule=_orig("fla_gdn")),
        "fla.ops": _stub("fla.ops"),
        "fla.ops.delta_rule": _stub("fla.ops.delta_rule", chunk_delta_rule=_orig("fla_op_dn")),
        "fla.ops.gated_delta_rule": _stub("fla.ops.gated_delta_rule",
                                          chunk_gated_delta_rule=_orig("fla_op_gdn")),
    }
    for name, m in mods.items():
        monkeypatch.setitem(sys.modules, name, m)
    yield mods
    patch.restore()


def test_patch_rebinds_every_name(stub_reference):
    m = stub_reference
    done = patch.apply()
    for n in KATA_NAMES:
        assert getattr(m["kata.parallel_kata_attn"], n) is getattr(parallel_kata_attn, n)
    for n in KATA_NAMES[:5]:
        assert getattr(m["kata.layer"], n) is getattr(parallel_kata_attn, n)
    # a name the mixer never imported is not added to it
    assert not hasattr(m["kata.layer"], "parallel_kata_attn_bwd")
    assert m["kata.spd.chunk_scan_cat"].spd_chunk_scan_cat is spd_state.spd_chunk_scan_cat
    from linatt_amd import flash_delta as fd, mixer
    for n in MIXER_NAMES:
        assert getattr(m["kata.layer"], n) is getattr(mixer, n)
    for n in DELTA_KATA_NAMES:
        assert getattr(m["kata.spd.flash_delta"], n) is getattr(fd, n)
    assert m["kata.layer"].flash_delta is fd.flash_delta
    assert m["fla.layers.delta_net"].chunk_delta_rule is delta_rule.chunk_delta_rule
    assert m["fla.ops.delta_rule"].chunk_delta_rule is delta_rule.chunk_delta_rule
    assert m["fla.layers.gated_deltanet"].chunk_gated_delta_rule is delta_rule.chunk_gated_delta_rule
    assert m["fla.ops.gated_delta_rule"].chunk_gated_delta_rule is delta_rule.chunk_gated_delta_rule
    assert len(done) == len(KATA_NAMES) + 5 + 5 + 4 + 1 + len(MIXER_NAMES)


def test_patch_is_idempotent_and_restorable(stub_reference):
    m = stub_reference
    first = patch.apply()
    second = patch.apply()
    assert first == second
    assert m["kata.layer"].parallel_kata_attn is parallel_kata_attn.parallel_kata_attn
    patch.restore()
    assert m["kata.layer"].parallel_kata_attn() == "layer_parallel_kata_attn"
    assert m["fla.layers.delta_net"].chunk_delta_rule() == "fla_dn"
    assert m["kata.parallel_kata_attn"].parallel_kata_attn_bwd() == "ref_parallel_kata_attn_bwd"


def test_patch_skips_absent_modules(monkeypatch):
    # no reference packages at all: nothing to rebind, and no error
    for name in [n for n in sys.modules if n == "kata" or n.startswith(("kata.", "fla"))]:
        monkeypatch.delitem(sys.modules, name)
    monkeypatch.setattr(sys, "path", [p for p in sys.path if "reference" not in p])
    assert patch.apply() == []


def _cpu(*shape, dtype=torch.bfloat16):
    return torch.zeros(*shape, dtype=dtype)


@pytest.mark.parametrize("fn", ["chunk_delta_rule", "chunk_gated_delta_rule"])
def test_delta_rule_refuses_head_first_and_unknown_kwargs(fn):
    q = _cpu(1, 8, 2, 64)
    beta = _cpu(1, 8, 2, dtype=torch.float32)
    args = (q, q, q, beta) if fn == "chunk_delta_rule" else (q, q, q, beta, beta)
    op = getattr(delta_rule, fn)
    with pytest.raises(NotImplementedError, match="head_first"):
        op(*args, head_first=True)
    with pytest.raises(TypeError, match="unexpected keyword"):
        op(*args, chunk_size=32)
    # varlen takes the same device check as every call: no CPU path
    with pytest.raises(RuntimeError, match="no CPU path"):
        op(*args, cu_seqlens=torch.tensor([0, 8]))


def test_decode_step_validates_shapes_before_launch():
    B, H, D = 2, 3, 64
    S = torch.zeros(B, H, 4 * 16 * 16, D)
    z = torch.zeros(B, H, 4 * 16 * 16)
    q = _cpu(B, H, D)
    with pytest.raises(ValueError, match="k must be"):
        spd_state.kata_decode_step(S, z, q, _cpu(B, 1, D), _cpu(B, H, D))
    with pytest.raises(ValueError, match="k must be"):
        spd_state.kata_decode_step(S, z, q, q, _cpu(B + 1, H, D))
    with pytest.raises(ValueError, match=r"\(B, H, dk\)"):
        spd_state.kata_decode_step(S, z, _cpu(B, 1, H, D), q, q)
    # well-formed CPU tensors still raise: there is no CPU path
    with pytest.raises(RuntimeError, match="no CPU path"):
        spd_state.kata_decode_step(S, z, q, q, _cpu(B, H, D))


# ---------------------------------------------------------------------------
# the decode cache's host logic (linatt_amd.kata_cache)
# ---------------------------------------------------------------------------


def test_layer_state_cache_contract():
    from linatt_amd.kata_cache import LayerStateCache, get_layer_cache, update_layer_cache

    class Layer:
        def __init__(self, i):
            self.layer_idx = i

    l0, l1 = Layer(0), Layer(1)
    assert get_layer_cache(l0, None) is None
    assert update_layer_cache(l0, None, recurrent_state=1) is None
    cache = LayerStateCache()
    assert get_layer_cache(l0, cache) is None and cache.get_seq_length() == 0
    update_layer_cache(l0, cache, recurrent_state="s0", conv_state="c0", offset=7)
    update_layer_cache(l1, cache, recurrent_state="s1", offset=7)
    assert len(cache) == 2 and cache.get_seq_length() == 7
    assert get_layer_cache(l0, cache)["recurrent_state"] == "s0"
    # a later update replaces only the entries it names
    update_layer_cache(l0, cache, recurrent_state="s0b", offset=1)
    assert cache[0] == {"recurrent_state": "s0b", "attn_state": None, "conv_state": "c0",
                        "ffn_state": None}
    assert cache.get_seq_length() == 8
    with pytest.raises(IndexError):
        cache.update(recurrent_state="x", layer_idx=5)


def test_cached_attention_validates_shapes():
    from linatt_amd.kata_cache import KataState, parallel_kata_attn_cached
    q = _cpu(2, 3, 4, 64)
    with pytest.raises(ValueError, match="q, k must be"):
        parallel_kata_attn_cached(q, _cpu(2, 3, 4, 32), q)
    st = KataState(torch.zeros(1, 4, 1024, 64), torch.zeros(1, 4, 1024), 10)
    with pytest.raises(ValueError, match="state is for"):
        parallel_kata_attn_cached(q, q, q, st)


def test_flash_delta_validates_before_launch():
    from linatt_amd import flash_delta as fd
    q = _cpu(1, 8, 2, 64)
    beta = _cpu(1, 8, 2, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="no CPU path"):
        fd.flash_delta(q, q, q, beta, 1)


# ---------------------------------------------------------------------------
# the fused mixer forward (linatt_amd.patch.apply_mixer)
# ---------------------------------------------------------------------------


@pytest.fixture
def mixer_hook(monkeypatch):
    """kata.layer as a stub module whose KataAttention has the reference's
    attribute layout, the hook installed on it, and the device ops the hook
    calls replaced by recorders (no GPU here): each returns tensors of the
    right shapes and logs its name."""
    import mixer_layout
    from linatt_amd import kata_cache, kata_layer

    class KataAttention(mixer_layout.KataAttentionLayout):
        pass

    mods = {"kata": _stub("kata"), "kata.layer": _stub("kata.layer", KataAttention=KataAttention)}
    for name, m in mods.items():
        monkeypatch.setitem(sys.modules, name, m)
    calls = []

    def prologue(x, conv, norm, rot, head_dim, seqlen_offset=0, cache=None, output_final_state=False):
        calls.append(("fused_qk_prologue", norm if isinstance(norm, (str, type(None))) else "rmsnorm",
                      seqlen_offset))
        B, T, C = x.shape
        st = torch.zeros(B, C, conv.weight.shape[-1]) if output_final_state else None
        return x.reshape(B, T, C // head_dim, head_dim), st

    def conv(x, w, b, act, cache, out_state):
        calls.append(("short_conv",))
        return x, (torch.zeros(x.shape[0], x.shape[-1], w.shape[-1]) if out_state else None)

    def onorm(q, k, v, w, eps, M, scale, variant, c):
        calls.append(("parallel_kata_attn_onorm", variant, c is not None, tuple(k.shape)))
        return torch.zeros(*q.shape[:3], v.shape[-1], dtype=v.dtype)

    def cached(q, k, v, state, M, scale, variant="concat", c=None):
        calls.append(("parallel_kata_attn_cached", state is not None, tuple(k.shape)))
        calls.append(("cached_score", variant, c is not None))
        off = 0 if state is None else state.offset
        return (torch.zeros(*q.shape[:3], v.shape[-1], dtype=v.dtype),
                kata_cache.KataState(None, None, off + q.shape[1]))

    def norm(x, w, eps):
        calls.append(("rms_norm",))
        return x

    monkeypatch.setattr(kata_layer, "fused_qk_prologue", prologue)
    monkeypatch.setattr(kata_layer, "short_conv", conv)
    monkeypatch.setattr(kata_layer, "parallel_kata_attn_onorm", onorm)
    monkeypatch.setattr(kata_layer.kata_cache, "parallel_kata_attn_cached", cached)
    monkeypatch.setattr(kata_layer, "rms_norm", norm)
    assert patch.apply_mixer()
    yield KataAttention, calls
    patch.restore()
    assert KataAttention.forward is mixer_layout.KataAttentionLayout.forward


def test_apply_mixer_reaches_prologue_epilogue_and_cache(mixer_hook):
    KataAttention, calls = mixer_hook
    from linatt_amd import kata_cache, kata_layer
    assert KataAttention.forward is kata_layer.kata_attention_forward
    assert patch.apply_mixer()  # idempotent
    layer = KataAttention(64, 4, 64, 4, num_kv_heads=2)
    x = torch.randn(2, 10, 64)
    out, _, pkv = layer(x)
    assert out.shape == (2, 10, 64) and pkv is None and layer.original_calls == 0
    assert [c[0] for c in calls] == ["short_conv", "fused_qk_prologue", "fused_qk_prologue",
                                     "parallel_kata_attn_onorm"]
    # GQA runs natively: k keeps its 2 kv heads
    assert calls[-1] == ("parallel_kata_attn_onorm", "concat", False, (2, 10, 2, 64))

    # with a cache: the state form, prefill then one decode step, the rotation
    # offset advancing and the convolution states kept for the next call
    # (bf16 projections, as under autocast: the state kernels are bf16)
    calls.clear()
    layer, x = layer.bfloat16(), x.bfloat16()
    cache = kata_cache.LayerStateCache()
    layer(x, past_key_values=cache, use_cache=True)
    layer(x[:, :1], past_key_values=cache, use_cache=True)
    names = [c[0] for c in calls]
    assert names.count("parallel_kata_attn_cached") == 2 and names.count("rms_norm") == 2
    assert [c for c in calls if c[0] == "parallel_kata_attn_cached"] == [
        ("parallel_kata_attn_cached", False, (2, 10, 4, 64)),   # k repeated to the 4 heads
        ("parallel_kata_attn_cached", True, (2, 1, 4, 64))]
    assert [c[2] for c in calls if c[0] == "fused_qk_prologue"] == [0, 0, 10, 10]
    assert cache.get_seq_length(0) == 11 and cache[0]["conv_state"] is not None
    assert cache[0]["recurrent_state"].offset == 11


@pytest.mark.parametrize("kw,expect", [
    (dict(feature_map="kata_quadratic_sum", norm_q="l2", norm_k="l2", rope_group=True),
     ("parallel_kata_attn_onorm", "sum", False)),
    (dict(use_decay=True), ("parallel_kata_attn_onorm", "concat", True)),
])
def test_apply_mixer_variants(mixer_hook, kw, expect):
    KataAttention, calls = mixer_hook
    layer = KataAttention(64, 4, 64, 2, **kw)
    layer(torch.randn(1, 5, 64))
    assert calls[-1][:3] == expect
    assert [c[1] for c in calls if c[0] == "fused_qk_prologue"] == (
        ["l2", "l2"] if kw.get("norm_q") == "l2" else ["rmsnorm", "rmsnorm"])


def test_apply_mixer_falls_back_outside_its_scope(mixer_hook):
    KataAttention, calls = mixer_hook
    from linatt_amd import kata_cache
    # a psi-feature map: the reference's own forward
    layer = KataAttention(64, 4, 64, 4, feature_map="positive")
    assert layer(torch.randn(1, 5, 64))[0][0] == "original" and layer.original_calls == 1
    # a cache for a shape with no state form (groups of 8 dims): the
    # reference's forward
    layer = KataAttention(64, 4, 64, 8).bfloat16()
    layer(torch.randn(1, 5, 64).bfloat16(), past_key_values=kata_cache.LayerStateCache(),
          use_cache=True)
    assert layer.original_calls == 1 and not calls


@pytest.mark.parametrize("kw,score", [
    (dict(feature_map="kata_quadratic_sum"), ("cached_score", "sum", False)),
    (dict(use_decay=True), ("cached_score", "concat", True)),
    (dict(use_offset_gate=True), ("cached_score", "concat", False)),
])
def test_apply_mixer_cache_for_every_flash_score(mixer_hook, kw, score):
    """Sum, decayed and offset-gated scores decode from a state too."""
    KataAttention, calls = mixer_hook
    from linatt_amd import kata_cache
    layer = KataAttention(64, 4, 64, 2, **kw).bfloat16()
    layer(torch.randn(1, 5, 64).bfloat16(), past_key_values=kata_cache.LayerStateCache(),
          use_cache=True)
    assert layer.original_calls == 0 and score in calls
