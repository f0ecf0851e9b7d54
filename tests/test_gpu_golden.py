"""The HIP path on the committed golden fixtures (``tests/golden``): each
case's stored inputs go through the product's operator API on ``cuda:0`` and
every output and gradient is compared with the stored float64-oracle values,
without running the oracle on the GPU box.  Bars as in the other GPU
parity tests: max|x - ref| / max|ref| below 2e-2 for bfloat16 inputs.
"""

import pytest
import torch

from golden import store

pytestmark = pytest.mark.gpu

BAR = 2e-2
MAN = store.manifest()


def mar(x, ref):
    x = x.detach().double().cpu()
    den = ref.abs().max().item()
    return (x - ref).abs().max().item() / (den if den > 0 else 1.0)


def _leaves(x, names):
    return {n: x[n].cuda().requires_grad_(True) for n in names}


def run_kata(x):
    from linatt_amd import parallel_kata_attn as P
    p = x["params"]
    L = _leaves(x, ("q", "k", "v"))
    concat = p["variant"] == "concat"
    fn = P.parallel_kata_attn if concat else P.parallel_kata_attn_sum
    o = fn(L["q"], L["k"], L["v"], num_groups=p["M"], scale=p["scale"])
    o.backward(x["do"].cuda())
    impl = P.parallel_kata_attn_fwd_impl if concat else P.parallel_kata_attn_sum_fwd_impl
    with torch.no_grad():
        _, den = impl(L["q"].detach(), L["k"].detach(), L["v"].detach(), p["M"], p["scale"], 64, 64)
    return {"o": o, "den": den, "dq": L["q"].grad, "dk": L["k"].grad, "dv": L["v"].grad}


def run_kata_decay(x):
    from linatt_amd import parallel_kata_attn as P
    p = x["params"]
    L = _leaves(x, ("q", "k", "v", "c"))
    o = P.parallel_kata_attn_decay(L["q"], L["k"], L["v"], L["c"], num_groups=p["M"], scale=p["scale"])
    o.backward(x["do"].cuda())
    return {"o": o, **{"d" + n: t.grad for n, t in L.items()}}


def run_delta(x):
    from linatt_amd import delta_rule as R
    names = [n for n in ("q", "k", "v", "beta", "g", "h0") if n in x]
    L = _leaves(x, names)
    kw = dict(scale=x["params"]["scale"], initial_state=L.get("h0"), output_final_state=True)
    if "g" in L:
        o, ht = R.chunk_gated_delta_rule(L["q"], L["k"], L["v"], L["g"], L["beta"], **kw)
    else:
        o, ht = R.chunk_delta_rule(L["q"], L["k"], L["v"], L["beta"], **kw)
    loss = (o.float() * x["do"].cuda().float()).sum()
    if "dht" in x:
        loss = loss + (ht * x["dht"].cuda()).sum()
    loss.backward()
    return {"o": o, "ht": ht, **{"d" + n: t.grad for n, t in L.items()}}


def run_kata_state(x):
    from linatt_amd import spd_state as S_
    p = x["params"]
    T = p["T"]
    q, k, v = (x[n].cuda() for n in ("q", "k", "v"))
    o, den, S, z = S_.kata_prefill(q[:, :T], k[:, :T], v[:, :T], num_groups=p["M"], eps=p["eps"],
                                   seg_len=p["seg_len"])
    got = {"o": o, "den": den, "S": S.clone(), "z": z.clone()}
    got["o_decode"] = S_.kata_decode_step(S, z, q[:, T].contiguous(), k[:, T].contiguous(),
                                          v[:, T].contiguous(), num_groups=p["M"], eps=p["eps"])
    got["z_decode"] = z
    return got


def run_flash_delta(x):
    from linatt_amd import flash_delta as F
    p = x["params"]
    L = _leaves(x, ("q", "k", "v", "beta"))
    o = F.flash_delta(L["q"], L["k"], L["v"], L["beta"], p["M"], scale=p["scale"])
    o.backward(x["do"].cuda())
    return {"o": o, **{"d" + n: t.grad for n, t in L.items()}}


def run_mixer(x):
    from linatt_amd import mixer as MX
    p = x["params"]
    L = _leaves(x, ("x", "w", "b"))
    y, _ = MX.short_conv(L["x"], L["w"], L["b"], "silu")
    y.backward(x["dy"].cuda())
    B, T, C = x["x"].shape
    Dh = p["head_dim"]
    xr = x["x"].reshape(B, T, C // Dh, Dh).cuda().requires_grad_(True)
    nw = x["nw"].cuda().requires_grad_(True)
    n = MX.rms_norm(xr, nw, p["eps"])
    n.backward(x["dy"].reshape(B, T, C // Dh, Dh).cuda())
    return {"conv_y": y, "conv_dx": L["x"].grad, "conv_dw": L["w"].grad, "conv_db": L["b"].grad,
            "norm_y": n, "norm_dx": xr.grad, "norm_dw": nw.grad}


RUN = {
    "kata_concat_m4_gqa": run_kata,
    "kata_sum_m2": run_kata,
    "kata_decay_dk128_m2": run_kata_decay,
    "delta_gated_h0": run_delta,
    "delta_k128": run_delta,
    "kata_state_m4": run_kata_state,
    "flash_delta_m2": run_flash_delta,
    "mixer": run_mixer,
}


def test_every_case_has_a_runner():
    assert sorted(RUN) == sorted(MAN)


@pytest.mark.parametrize("name", sorted(MAN))
def test_hip_path_matches_fixture(name):
    print(f"\ngolden case {name}", flush=True)
    x, out = store.load(name, MAN[name])
    got = RUN[name](x)
    torch.cuda.synchronize()
    assert sorted(got) == sorted(out), (sorted(got), sorted(out))
    errs = {n: mar(got[n], ref) for n, ref in out.items()}
    print(errs, flush=True)
    for n, ref in out.items():
        assert tuple(got[n].shape) == tuple(ref.shape), n
        assert errs[n] < BAR, (n, errs[n])
