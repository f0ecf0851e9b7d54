"""CPU checks of the committed golden fixtures (``tests/golden``).

* every ``.npz`` matches the sha256 its manifest records;
* the stored inputs are exactly what the seeded recipe draws, so a fixture
  can be regenerated and compared bit for bit;
* the oracle, run again on the stored inputs, reproduces the stored outputs
  to the float32 rounding of the file (a regression guard: a change to the
  oracle that moves any of these numbers fails here);
* the comparison has teeth: a plausible mistake planted in the oracle's
  call (the other score variant, a wrong number of groups, the decay sign,
  the gate dropped) moves the outputs far beyond the bar.
"""

import pytest
import torch

from golden import cases, store

MAN = store.manifest()


def rel(x, ref):
    den = ref.abs().max().item()
    return (x.double() - ref).abs().max().item() / (den if den > 0 else 1.0)


def test_manifest_lists_every_case():
    assert sorted(MAN) == sorted(cases.CASES)


@pytest.mark.parametrize("name", sorted(cases.CASES))
def test_fixture_digest_and_inputs(name):
    entry = MAN[name]
    assert store.sha256(store.path(name)) == entry["sha256"], "fixture file changed"
    make_in, _, seed = cases.CASES[name]
    assert entry["seed"] == seed
    x, out = store.load(name, entry)
    fresh = make_in(seed)
    assert fresh["params"] == x["params"]
    for n, t in fresh.items():
        if n == "params":
            continue
        assert t.dtype == x[n].dtype and torch.equal(t, x[n]), n
    assert sorted(out) == sorted(entry["outputs"])
    for n, t in out.items():
        assert list(t.shape) == entry["outputs"][n] and torch.isfinite(t).all(), n


@pytest.mark.parametrize("name", sorted(cases.CASES))
def test_oracle_reproduces_fixture(name):
    _, make_out, _ = cases.CASES[name]
    x, out = store.load(name)
    got = make_out(x)
    assert sorted(got) == sorted(out)
    for n, ref in out.items():
        assert got[n].shape == ref.shape, n
        e = rel(got[n], ref)
        assert e < 1e-6, (n, e)


def _planted(name, x):
    """The case recomputed with one plausible mistake in the oracle's call."""
    p = dict(x["params"])
    if name == "kata_concat_m4_gqa":
        p["variant"] = "sum"
        return cases.kata_out({**x, "params": p})
    if name == "kata_sum_m2":
        p["M"] = 4
        return cases.kata_out({**x, "params": p})
    if name == "kata_decay_dk128_m2":
        return cases.kata_decay_out({**x, "c": -x["c"]})
    if name == "delta_gated_h0":
        return cases.delta_out({n: t for n, t in x.items() if n != "g"})
    if name == "delta_k128":
        return cases.delta_out({**x, "k": x["k"].flip(1)})
    if name == "kata_state_m4":
        p["M"] = 2
        return cases.kata_state_out({**x, "params": p})
    if name == "flash_delta_m2":
        p["M"] = 1
        return cases.flash_delta_out({**x, "params": p})
    if name == "mixer":
        return cases.mixer_out({**x, "w": x["w"].flip(-1)})
    raise KeyError(name)


@pytest.mark.parametrize("name", sorted(cases.CASES))
def test_fixture_detects_planted_mistake(name):
    x, out = store.load(name)
    got = _planted(name, x)
    worst = max(rel(got[n], out[n]) for n in out if n in got and got[n].shape == out[n].shape)
    assert worst > 5e-2, worst
