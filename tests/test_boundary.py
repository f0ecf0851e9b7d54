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
